"""GPU parity of every C-ABI entry point against the CPU oracle (same seeded inputs).

Gates (north star): fp32 paths within 1e-4 normwise of the oracle's fp32
results and within 1e-2 elementwise (tests/helpers.py: |a - r| / max(|r|,
1e-3 rms(r)), bounded above the reference order's own fp32 rounding noise);
fp16 paths within 2e-2 normwise of the fp32 oracle (they are
also checked against the oracle's fp16-storage mode, which mirrors the
reference's own fp16 rounding points).  Integer work (dropout masks) must be
bit-exact.
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


def make_pair(ctx, K, N, M, seed, *, half=False, norm=0, act=0, leaky=0.0, p=0.0, bias_sigma=0.01,
              regularisation=0, regu_coeff=0.0):
    g = rng(seed)
    w = he_normal(g, K, N)
    b = (g.standard_normal((1, N)) * bias_sigma).astype(np.float32)
    if half:
        b = f16(b)
    kw = dict(half=half, norm=norm, act=act, leaky=leaky, mask_coeff=p, regularisation=regularisation,
              regu_coeff=regu_coeff, b=b)
    # fp16 blocks follow the convert_f16 route: master = fp32 original, w = RNE(master)
    ob = O.OracleBlock(K, N, M, w, master_w=w if half else None, **kw)
    db = DeviceBlock(ctx, K, N, M, w, master_w=w if half else None, **kw)
    return ob, db


def dev(x: np.ndarray, half: bool) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(torch.float16 if half else torch.float32)


def inputs(seed, M, K, half, scale=1.0):
    x = (rng(seed).standard_normal((M, K)) * scale).astype(np.float32)
    return f16(x) if half else x


# ---------------------------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------------------------
FWD_CASES = [
    # (M, K, N, norm, act, dropout p)
    (256, 192, 160, 0, 2, 0.0),     # ReLU, vector path
    (512, 256, 384, 0, 6, 0.0),     # SiLU
    (37, 45, 29, 0, 7, 0.0),        # Mish, ragged (element-wise staging)
    (128, 96, 64, 1, 7, 0.1),       # RMSNorm + Mish + dropout
    (96, 80, 144, 2, 3, 0.2),       # LayerNorm + LeakyReLU + dropout
    (64, 48, 40, 3, 4, 0.0),        # BatchNorm + Tanh
    (33, 17, 11, 2, 1, 0.0),        # LN + Sigmoid, ragged
    # widths that are not a multiple of 4: rows start at every offset within
    # a 4-element group (the aligned-group norm kernel, 1..4 groups per thread)
    (301, 64, 1531, 2, 3, 0.1),     # LN + LeakyReLU + dropout
    (130, 40, 3001, 1, 7, 0.0),     # RMSNorm + Mish
    (70, 32, 1022, 2, 6, 0.0),      # LN + SiLU, width 2 mod 4
    (50, 24, 4093, 1, 4, 0.2),      # RMSNorm + Tanh + dropout, 4 groups per thread
    # outputs of <= 16 columns (the skinny forward): odd K (rows not 16-byte
    # aligned, a partial last k-chunk), a partial last block of 16 rows, dropout;
    # and K a multiple of 8 (16-byte row loads) over several rounds of row blocks
    (1000, 3001, 13, 0, 1, 0.1),    # Sigmoid + dropout
    (4100, 2048, 10, 0, 2, 0.0),    # ReLU
    # ragged 256x256 path at C5's first-layer shape (294 tiles, padded operands,
    # element-wise epilogue) with the fused activation and dropout
    (12345, 777, 1531, 0, 6, 0.1),  # SiLU + dropout
]


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("M,K,N,norm,act,p", FWD_CASES)
def test_forward(ctx, half, M, K, N, norm, act, p):
    ob, db = make_pair(ctx, K, N, M, seed=M + K + N, half=half, norm=norm, act=act, leaky=0.01, p=p)
    x = inputs(7, M, K, half)
    seed = O.scramble_seed(3, 11)
    ob.forward(x, M, p > 0, seed)
    db.forward(dev(x, half), M, p > 0, seed)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    names = ["preact", "predrop", "out"] + (["prenorm", "centered"] if norm else [])
    for n in names:
        check(n, db.get(n)[:M], getattr(ob, n)[:M], tol)
    if norm:
        rows = N if norm == 3 else M
        check("norm_rstd", db.get("norm_rstd")[:rows], ob.norm_rstd[:rows], tol)
    if p > 0:
        assert np.array_equal(db.get("mask")[:M], ob.mask[:M]), "dropout mask differs"


@pytest.mark.parametrize("M,K,N,norm,act", [(256, 192, 160, 0, 6), (96, 80, 144, 2, 3), (64, 48, 40, 1, 7)])
def test_forward_fp16_vs_fp32_oracle(ctx, M, K, N, norm, act):
    """fp16 path against the pure fp32 oracle on the same (f16-representable) inputs."""
    g = rng(5)
    w = f16(he_normal(g, K, N))
    x = inputs(8, M, K, True)
    o32 = O.OracleBlock(K, N, M, w, norm=norm, act=act, leaky=0.01)
    db = DeviceBlock(ctx, K, N, M, w, half=True, norm=norm, act=act, leaky=0.01)
    o32.forward(x, M)
    db.forward(dev(x, True), M)
    torch.cuda.synchronize()
    check("out", db.get("out")[:M], o32.out[:M], FP16_TOL)


# ---------------------------------------------------------------------------------------------
# output error (+ softmax)
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("loss,act,norm", [(abi.LOSS_CE, abi.ACT_SOFTMAX, 0), (abi.LOSS_BCE, abi.ACT_SIGMOID, 2),
                                           (abi.LOSS_MSE, abi.ACT_IDENTITY, 1), (abi.LOSS_MSE, abi.ACT_SIGMOID, 0)])
def test_output_error(ctx, half, loss, act, norm):
    M, K, N = 64, 48, 10
    ob, db = make_pair(ctx, K, N, M, seed=11, half=half, norm=norm)
    x = inputs(12, M, K, half)
    ob.forward(x, M)
    db.forward(dev(x, half), M)
    lab = rng(13).integers(0, N, M)
    t = np.zeros((M, N), np.float32)
    t[np.arange(M), lab] = 1.0
    ob.output_error(t, loss, act)
    db.output_error(dev(t, half), loss, act)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    check("out(after loss act)", db.get("out"), ob.out, tol)
    check("grad", db.get("grad"), ob.grad, tol)
    check("d_prenorm", db.get("d_prenorm"), ob.d_prenorm, tol)
    if norm:
        check("d_norm_w", db.get("d_norm_w"), ob.d_norm_w, tol)
    if half:
        assert np.array_equal(db.get("d_prenorm_h"), f16(db.get("d_prenorm")))


# ---------------------------------------------------------------------------------------------
# hidden error (dX GEMM + act' + mask + norm gradient)
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("M,K0,N0,N1,norm,act,p", [(128, 64, 96, 80, 0, 6, 0.0), (96, 40, 72, 24, 2, 3, 0.1),
                                                   (77, 33, 51, 13, 1, 7, 0.0), (256, 128, 256, 192, 0, 2, 0.0),
                                                   (66, 24, 40, 6, 3, 3, 0.0)])
def test_hidden_error(ctx, half, M, K0, N0, N1, norm, act, p):
    """Next layers of up to 16 outputs (N1 13, 6) take the error kernel that forms the sum itself."""
    o0, d0 = make_pair(ctx, K0, N0, M, seed=21, half=half, norm=norm, act=act, leaky=0.01, p=p)
    o1, d1 = make_pair(ctx, N0, N1, M, seed=22, half=half, act=abi.ACT_IDENTITY)
    x = inputs(23, M, K0, half)
    seed = 12345
    o0.forward(x, M, p > 0, seed)
    d0.forward(dev(x, half), M, p > 0, seed)
    o1.forward(o0.out, M)
    d1.forward(d0.out, M)
    t = (rng(24).random((M, N1)) > 0.5).astype(np.float32)
    o1.output_error(t, abi.LOSS_BCE, abi.ACT_SIGMOID)
    d1.output_error(dev(t, half), abi.LOSS_BCE, abi.ACT_SIGMOID)
    o0.hidden_error(o1, M)
    d0.hidden_error(d1, M)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    check("grad", d0.get("grad")[:M], o0.grad[:M], tol)
    check("d_prenorm", d0.get("d_prenorm")[:M], o0.d_prenorm[:M], tol)
    if norm:
        check("d_norm_w", d0.get("d_norm_w")[:M], o0.d_norm_w[:M], tol)
        check("d_norm_b", d0.get("d_norm_b")[:M], o0.d_norm_b[:M], tol)


# ---------------------------------------------------------------------------------------------
# error from a supplied sum + input gradient
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("M,K,N,norm,act", [(256, 192, 160, 0, 6), (45, 37, 29, 2, 3)])
def test_error_from_sum_and_input_grad(ctx, half, M, K, N, norm, act):
    ob, db = make_pair(ctx, K, N, M, seed=31, half=half, norm=norm, act=act, leaky=0.01)
    x = inputs(32, M, K, half)
    ob.forward(x, M)
    db.forward(dev(x, half), M)
    s = (rng(33).standard_normal((M, N)) * 512).astype(np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    dx = db.input_grad(M)
    torch.cuda.synchronize()
    tol = FP16_TOL if half else FP32_TOL
    check("grad", db.get("grad")[:M], ob.grad[:M], tol)
    check("d_prenorm", db.get("d_prenorm")[:M], ob.d_prenorm[:M], tol)
    check("input_grad", dx.cpu().numpy(), ob.input_grad(M), tol)


# ---------------------------------------------------------------------------------------------
# backward: dW / db / norm sums + optimiser
# ---------------------------------------------------------------------------------------------
def _run_backward(ctx, half, M, K, N, norm, opt_kind, step=1, regularisation=0, regu_coeff=0.0, lr=0.01,
                  call_between=False):
    ob, db = make_pair(ctx, K, N, M, seed=41 + M, half=half, norm=norm, act=abi.ACT_SILU,
                       regularisation=regularisation, regu_coeff=regu_coeff)
    x = inputs(42, M, K, half)
    ob.forward(x, M)
    db.forward(dev(x, half), M)
    s = (rng(43).standard_normal((M, N)) * 512).astype(np.float32)
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    if call_between == "input_grad":
        # dX between the error and the backward call (a single block's order): it leaves
        # d_prenorm / dNorm alone, so the backward keeps the error call's column sums
        ob.input_grad(M)
        db.input_grad(M)
    elif call_between == "input_grad_into_d_prenorm":
        # dx written over d_prenorm (K == N): the backward must sum the overwritten
        # d_prenorm, as the reference's backward reads whatever the buffer holds
        ob.d_prenorm[:M] = ob.input_grad(M)
        db.input_grad(M, out=db.d_prenorm[:M])
    elif call_between:
        # any other entry point between the error and the backward call: the backward then
        # sums d_prenorm / dNorm over the rows itself instead of using the error call's sums
        ctx.synchronize()
    if opt_kind == abi.OPT_SGD:
        oo, do = O.Optimiser.sgd(0.0), abi.sgd(0.0)
    else:
        oo, do = O.Optimiser.adam(0.9, 0.999, 1e-8), abi.adam(0.9, 0.999, 1e-8)
    ob.backward(x, oo, oo, M, lr, 3.4e38, step)
    db.backward(dev(x, half), abi.train_ctx(do, do, M, lr), step)
    torch.cuda.synchronize()
    return ob, db


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("M,K,N,norm", [(256, 128, 160, 0), (512, 64, 64, 2), (123, 77, 45, 1), (40, 24, 16, 3),
                                        (2048, 256, 256, 0)])
def test_backward_sgd(ctx, half, M, K, N, norm):
    """SGD with v = 0 leaves the batch-mean gradient in dv (backward.cu:127-128)."""
    ob, db = _run_backward(ctx, half, M, K, N, norm, abi.OPT_SGD)
    tol = FP16_TOL if half else FP32_TOL
    check("dv_w (= dW / 512 / m)", db.get("dv_w"), ob.dv_w, tol)
    mw = "master_w" if half else "w"
    check("W after step", db.get(mw), getattr(ob, mw), tol)
    if norm != 3:
        check("dv_b (= db)", db.get("dv_b"), ob.dv_b, tol)
    if norm:
        check("dv_norm_w", db.get("dv_norm_w"), ob.dv_norm_w, tol)
    if norm > 1:
        check("dv_norm_b", db.get("dv_norm_b"), ob.dv_norm_b, tol)
    if half:
        assert np.array_equal(db.get("w"), f16(db.get("master_w"))), "w must equal f16(master_w)"


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("norm", [0, 1, 2])
@pytest.mark.parametrize("call_between", [False, True, "input_grad", "input_grad_into_d_prenorm"])
def test_backward_column_sums_from_error_call_or_recomputed(ctx, half, norm, call_between):
    """db and the dNorm sums come from the error call's own pass over the rows when the
    backward directly follows it (or follows a dX call that leaves the buffers alone), and
    are recomputed otherwise; all match the oracle."""
    K = 200 if call_between == "input_grad_into_d_prenorm" else 96
    ob, db = _run_backward(ctx, half, 320, K, 200, norm, abi.OPT_SGD, call_between=call_between)
    tol = FP16_TOL if half else FP32_TOL
    check("dv_b (= db)", db.get("dv_b"), ob.dv_b, tol)
    if norm:
        check("dv_norm_w", db.get("dv_norm_w"), ob.dv_norm_w, tol)
    if norm > 1:
        check("dv_norm_b", db.get("dv_norm_b"), ob.dv_norm_b, tol)


def test_backward_column_sums_not_taken_from_another_block(ctx):
    """Error calls on blocks A then B, backward on A: A's bias gradient must come from A's
    own d_prenorm, not from the column sums B's error call left behind."""
    M, K, N = 192, 64, 128
    oa, da = make_pair(ctx, K, N, M, seed=61, act=abi.ACT_SILU)
    ob_, db_ = make_pair(ctx, K, N, M, seed=62, act=abi.ACT_SILU)
    x = inputs(63, M, K, False)
    for o, d, sd in ((oa, da, 64), (ob_, db_, 65)):
        o.forward(x, M)
        d.forward(dev(x, False), M)
        s = (rng(sd).standard_normal((M, N)) * 512).astype(np.float32)
        o.error_from_sum(s, M)
        d.error_from_sum(torch.from_numpy(s).cuda(), M)
    oa.backward(x, O.Optimiser.sgd(0.0), O.Optimiser.sgd(0.0), M, 0.01, 3.4e38, 1)
    da.backward(dev(x, False), abi.train_ctx(abi.sgd(0.0), abi.sgd(0.0), M, 0.01), 1)
    torch.cuda.synchronize()
    check("dv_b (= db of block A)", da.get("dv_b"), oa.dv_b, FP32_TOL)


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("M,K,N,step", [(256, 128, 160, 1), (300, 100, 60, 7)])
def test_backward_adam(ctx, half, M, K, N, step):
    ob, db = _run_backward(ctx, half, M, K, N, 2, abi.OPT_ADAM, step=step, lr=1e-3)
    tol = FP16_TOL if half else FP32_TOL
    check("dm_w", db.get("dm_w"), ob.dm_w, tol)
    check("dv_w", db.get("dv_w"), ob.dv_w, tol)
    check("dm_b", db.get("dm_b"), ob.dm_b, tol)
    # the step itself, from the device's own moments (backward.cu:136-147)
    dm, dv = db.get("dm_w").astype(np.float64), db.get("dv_w").astype(np.float64)
    mhat = dm / (1 - 0.9 ** step)
    vhat = dv / (1 - 0.999 ** step)
    w0 = he_normal(rng(41 + M), K, N).astype(np.float64)
    expect = w0 - 1e-3 * mhat / (np.sqrt(vhat) + 1e-8)
    got = db.get("master_w" if half else "w")
    assert np.max(np.abs(got - expect)) < 1e-6


@pytest.mark.parametrize("regularisation,coeff", [(1, 1e-3), (2, 1e-2)])
def test_backward_regularisation(ctx, regularisation, coeff):
    ob, db = _run_backward(ctx, False, 128, 64, 48, 0, abi.OPT_SGD, regularisation=regularisation,
                           regu_coeff=coeff)
    check("W after step", db.get("w"), ob.w, FP32_TOL)


def test_backward_sgd_nesterov_momentum(ctx):
    M, K, N = 128, 64, 48
    ob, db = make_pair(ctx, K, N, M, seed=51, act=abi.ACT_RELU)
    x = inputs(52, M, K, False)
    for step in (1, 2, 3):
        ob.forward(x, M)
        db.forward(dev(x, False), M)
        s = (rng(53 + step).standard_normal((M, N)) * 512).astype(np.float32)
        ob.error_from_sum(s, M)
        db.error_from_sum(torch.from_numpy(s).cuda(), M)
        ob.backward(x, O.Optimiser.sgd(0.9, True), O.Optimiser.sgd(0.9, True), M, 0.05, 0.02, step)
        db.backward(dev(x, False), abi.train_ctx(abi.sgd(0.9, True), abi.sgd(0.9, True), M, 0.05, 0.02), step)
    torch.cuda.synchronize()
    check("W", db.get("w"), ob.w, FP32_TOL)
    check("dv_w", db.get("dv_w"), ob.dv_w, FP32_TOL)
