"""The C ABI's validation surface.

Each entry point repeats the reference's host-side checks, in the reference's
order, and returns one status per Error variant (src/util/log.rs:15-99):
DenseBlock::forward (src/mlp.rs:548-575, check_input_dimension at :492-519),
compute_loss (:756-811), backward_output (:607-639), backward_hidden
(:682-726), check_tile_dim (src/io/device.rs:248-258, run by gpu_forward_pass
and gpu_hidden_layer_backward_pass only: ffn_device.rs:20, 369) and
gpu_cast_t (src/io/device/util_device.rs:7-32).  Every misuse below must
return its code and leave every buffer of every block untouched (the buffers
hold a random pattern beforehand); the calls the reference lets through (no
tile_dim check on the output layer) must succeed.  skl_cast is also checked
bit for bit against IEEE round-to-nearest-even (numpy) in both directions.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import torch

from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock, F32_FIELDS, T_FIELDS
from tests.helpers import he_normal, rng

pytestmark = pytest.mark.gpu

OK = 0
INVALID_CONFIG, TRAINING_REQUIRED, ALLOC_LIMIT, MISMATCHED, BAD_BATCH, HW_CONSTRAINT = -1, -2, -3, -4, -5, -6
NULL_POINTER, UNSUPPORTED_CAST, NO_DEVICE = -8, -9, -10
FIELDS = T_FIELDS + F32_FIELDS + ("d_prenorm_h",)


@pytest.fixture(scope="module")
def ctx8(ctx):
    """A context created with tile_dim 8: the reference rejects fp16 launches of the forward and
    hidden-layer backward on it (check_tile_dim)."""
    c = abi.Context(0, 8)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    yield c
    torch.cuda.synchronize()
    c.close()


def block(ctx, K=32, N=48, M=64, *, half=False, seed=1, **kw):
    w = he_normal(rng(seed), K, N)
    db = DeviceBlock(ctx, K, N, M, w, half=half, master_w=w if half else None, **kw)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    for n in FIELDS:
        t = getattr(db, n)
        if t is not None:
            t.copy_(torch.randn(t.shape, generator=gen, device="cuda", dtype=torch.float32).to(t.dtype))
    torch.cuda.synchronize()
    return db


def snap(*blocks):
    torch.cuda.synchronize()
    return [{n: getattr(b, n).clone() for n in FIELDS if getattr(b, n) is not None} for b in blocks]


def assert_untouched(before, *blocks):
    torch.cuda.synchronize()
    for i, (s, b) in enumerate(zip(before, blocks)):
        for n, t in s.items():
            assert torch.equal(getattr(b, n), t), f"block {i}: {n} was written by a call that failed validation"


def xin(rows, cols, half):
    return torch.randn((max(rows, 1), cols), device="cuda").to(torch.float16 if half else torch.float32)


def st(name, *args):
    rc = abi.status(name, *args)
    torch.cuda.synchronize()
    return rc


def fwd(ctx, db, x, rows, cols, batch):
    return st("skl_dense_forward", ctx.h, C.byref(db.desc()), C.c_void_p(x.data_ptr()), rows, cols, batch, 0, 0)


def bwd(ctx, db, x, rows, cols, batch):
    tc = abi.train_ctx(abi.adam(), abi.adam(), batch, 1e-3)
    return st("skl_dense_backward", ctx.h, C.byref(db.desc()), C.c_void_p(x.data_ptr()), rows, cols,
              C.byref(tc), 1)


def bwd_hidden(ctx, cur, nxt, x, rows, cols, batch):
    tc = abi.train_ctx(abi.adam(), abi.adam(), batch, 1e-3)
    return st("skl_dense_backward_hidden", ctx.h, C.byref(cur.desc()), C.byref(nxt.desc()),
              C.c_void_p(x.data_ptr()), rows, cols, C.byref(tc), 1)


# ---- DenseBlock::forward (mlp.rs:548-575) ----------------------------------------------------
# (case, in_rows, in_cols, batch, block kwargs, expected)
FORWARD = [
    ("input rows < batch (mlp.rs:493-499)", 30, 32, 31, {}, MISMATCHED),
    ("input rows > max_batch (mlp.rs:501-507)", 65, 32, 64, {}, ALLOC_LIMIT),
    ("input cols != inputs (mlp.rs:509-516)", 64, 33, 64, {}, MISMATCHED),
    ("Softmax activation (mlp.rs:558-563)", 64, 32, 64, dict(act=abi.ACT_SOFTMAX), INVALID_CONFIG),
    ("batch 0 (mlp.rs:565-569)", 0, 32, 0, {}, BAD_BATCH),
    ("BatchNorm with batch 1 (mlp.rs:571-575)", 4, 32, 1, dict(norm=abi.NORM_BATCH), BAD_BATCH),
]


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("case", FORWARD, ids=[c[0] for c in FORWARD])
def test_forward_rejects(ctx, case, half):
    _, rows, cols, batch, kw, code = case
    db = block(ctx, half=half, **kw)
    x = xin(rows, cols, half)
    before = snap(db)
    assert fwd(ctx, db, x, rows, cols, batch) == code
    assert_untouched(before, db)


def test_forward_tile_dim(ctx8):
    """fp16 forward on a context whose tile_dim is not 16: HardwareConstraintViolation
    (ffn_device.rs:20); fp32 blocks do not care; the mlp.rs checks come first."""
    db = block(ctx8, half=True)
    x = xin(64, 32, True)
    before = snap(db)
    assert fwd(ctx8, db, x, 64, 32, 64) == HW_CONSTRAINT
    assert_untouched(before, db)
    sm = block(ctx8, half=True, act=abi.ACT_SOFTMAX)
    before = snap(sm)
    assert fwd(ctx8, sm, x, 64, 32, 64) == INVALID_CONFIG
    assert_untouched(before, sm)
    f32 = block(ctx8, half=False)
    assert fwd(ctx8, f32, xin(64, 32, False), 64, 32, 64) == OK


def test_forward_null_input(ctx):
    db = block(ctx)
    before = snap(db)
    assert st("skl_dense_forward", ctx.h, C.byref(db.desc()), None, 64, 32, 64, 0, 0) == NULL_POINTER
    assert_untouched(before, db)


# ---- compute_loss (mlp.rs:756-811) -------------------------------------------------------------
# (case, target rows, target cols, loss, loss activation, block kwargs, expected)
LOSS = [
    ("inference block (mlp.rs:762-766)", 64, 48, abi.LOSS_MSE, abi.ACT_IDENTITY, dict(is_training=False),
     TRAINING_REQUIRED),
    ("target cols (mlp.rs:768-774)", 64, 47, abi.LOSS_MSE, abi.ACT_IDENTITY, {}, MISMATCHED),
    ("target rows > max_batch (mlp.rs:776-782)", 65, 48, abi.LOSS_MSE, abi.ACT_IDENTITY, {}, ALLOC_LIMIT),
    ("MSE with Softmax (mlp.rs:785-792)", 64, 48, abi.LOSS_MSE, abi.ACT_SOFTMAX, {}, INVALID_CONFIG),
    ("CE without Softmax (mlp.rs:793-800)", 64, 48, abi.LOSS_CE, abi.ACT_SIGMOID, {}, INVALID_CONFIG),
    ("BCE without Sigmoid (mlp.rs:801-809)", 64, 48, abi.LOSS_BCE, abi.ACT_SOFTMAX, {}, INVALID_CONFIG),
]


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("case", LOSS, ids=[c[0] for c in LOSS])
def test_output_error_rejects(ctx, case, half):
    _, rows, cols, loss, act, kw, code = case
    db = block(ctx, half=half, **kw)
    t = xin(rows, cols, half)
    before = snap(db)
    assert st("skl_dense_output_error", ctx.h, C.byref(db.desc()), C.c_void_p(t.data_ptr()), rows, cols,
              loss, act, 0.0) == code
    assert_untouched(before, db)


def test_output_layer_ignores_tile_dim(ctx8):
    """gpu_compute_output_layer_error and gpu_backward_pass do not call check_tile_dim: an fp16
    output layer trains on a context with tile_dim 8."""
    db = block(ctx8, half=True)
    t = xin(64, 48, True)
    x = xin(64, 32, True)
    assert st("skl_dense_output_error", ctx8.h, C.byref(db.desc()), C.c_void_p(t.data_ptr()), 64, 48,
              abi.LOSS_MSE, abi.ACT_IDENTITY, 0.0) == OK
    assert bwd(ctx8, db, x, 64, 32, 64) == OK


# ---- backward_output (mlp.rs:607-639) ----------------------------------------------------------
BACKWARD = [
    ("inference block (mlp.rs:614-618)", 64, 32, 64, dict(is_training=False), TRAINING_REQUIRED),
    ("input rows < batch (mlp.rs:620)", 30, 32, 31, {}, MISMATCHED),
    ("input rows > max_batch (mlp.rs:620)", 65, 32, 64, {}, ALLOC_LIMIT),
    ("input cols != inputs (mlp.rs:620)", 64, 33, 64, {}, MISMATCHED),
    ("Softmax activation (mlp.rs:622-627)", 64, 32, 64, dict(act=abi.ACT_SOFTMAX), INVALID_CONFIG),
    ("batch 0 (mlp.rs:629-633)", 0, 32, 0, {}, BAD_BATCH),
    ("BatchNorm with batch 1 (mlp.rs:635-639)", 4, 32, 1, dict(norm=abi.NORM_BATCH), BAD_BATCH),
]


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("case", BACKWARD, ids=[c[0] for c in BACKWARD])
def test_backward_rejects(ctx, case, half):
    _, rows, cols, batch, kw, code = case
    db = block(ctx, half=half, **kw)
    x = xin(rows, cols, half)
    before = snap(db)
    assert bwd(ctx, db, x, rows, cols, batch) == code
    assert_untouched(before, db)


def test_backward_null_train_ctx(ctx):
    db = block(ctx)
    x = xin(64, 32, False)
    before = snap(db)
    assert st("skl_dense_backward", ctx.h, C.byref(db.desc()), C.c_void_p(x.data_ptr()), 64, 32, None, 1) \
        == NULL_POINTER
    assert_untouched(before, db)


# ---- backward_hidden (mlp.rs:682-726) ----------------------------------------------------------
# (case, in_rows, in_cols, batch, cur kwargs, next (inputs, max_batch), expected)
HIDDEN = [
    ("inference block (mlp.rs:682-686)", 64, 32, 64, dict(is_training=False), (48, 64), TRAINING_REQUIRED),
    ("input rows < batch (mlp.rs:688)", 30, 32, 31, {}, (48, 64), MISMATCHED),
    ("input rows > max_batch (mlp.rs:688)", 65, 32, 64, {}, (48, 64), ALLOC_LIMIT),
    ("input cols != inputs (mlp.rs:688)", 64, 33, 64, {}, (48, 64), MISMATCHED),
    ("next rows != cur cols (mlp.rs:690-697)", 64, 32, 64, {}, (40, 64), MISMATCHED),
    ("next grad rows < input rows (mlp.rs:699-706)", 48, 32, 32, {}, (48, 32), MISMATCHED),
    ("Softmax activation (mlp.rs:708-713)", 64, 32, 64, dict(act=abi.ACT_SOFTMAX), (48, 64), INVALID_CONFIG),
    ("batch 0 (mlp.rs:715-719)", 0, 32, 0, {}, (48, 64), BAD_BATCH),
    ("BatchNorm with batch 1 (mlp.rs:721-726)", 4, 32, 1, dict(norm=abi.NORM_BATCH), (48, 64), BAD_BATCH),
]


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("case", HIDDEN, ids=[c[0] for c in HIDDEN])
def test_backward_hidden_rejects(ctx, case, half):
    _, rows, cols, batch, kw, (n_in, n_m), code = case
    cur = block(ctx, half=half, **kw)
    nxt = block(ctx, K=n_in, N=24, M=n_m, half=half, seed=2)
    x = xin(rows, cols, half)
    before = snap(cur, nxt)
    assert bwd_hidden(ctx, cur, nxt, x, rows, cols, batch) == code
    assert_untouched(before, cur, nxt)


def test_backward_hidden_tile_dim(ctx8):
    """fp16 hidden-layer backward on tile_dim 8: HardwareConstraintViolation (ffn_device.rs:369), after
    the mlp.rs checks (a Softmax block still reports InvalidConfiguration); the same for the hidden
    error alone."""
    cur = block(ctx8, half=True)
    nxt = block(ctx8, K=48, N=24, half=True, seed=2)
    x = xin(64, 32, True)
    before = snap(cur, nxt)
    assert bwd_hidden(ctx8, cur, nxt, x, 64, 32, 64) == HW_CONSTRAINT
    assert st("skl_dense_hidden_error", ctx8.h, C.byref(cur.desc()), C.byref(nxt.desc()), 64) == HW_CONSTRAINT
    assert_untouched(before, cur, nxt)
    sm = block(ctx8, half=True, act=abi.ACT_SOFTMAX)
    before = snap(sm, nxt)
    assert bwd_hidden(ctx8, sm, nxt, x, 64, 32, 64) == INVALID_CONFIG
    assert_untouched(before, sm, nxt)


def test_hidden_error_rejects(ctx):
    cur = block(ctx)
    bad = block(ctx, K=40, N=24, seed=2)
    inf = block(ctx, is_training=False)
    nxt = block(ctx, K=48, N=24, seed=3)
    before = snap(cur, bad, inf, nxt)
    assert st("skl_dense_hidden_error", ctx.h, C.byref(cur.desc()), C.byref(bad.desc()), 64) == MISMATCHED
    assert st("skl_dense_hidden_error", ctx.h, C.byref(inf.desc()), C.byref(nxt.desc()), 64) == TRAINING_REQUIRED
    assert st("skl_dense_hidden_error", ctx.h, C.byref(cur.desc()), C.byref(nxt.desc()), 65) == ALLOC_LIMIT
    assert_untouched(before, cur, bad, inf, nxt)


# ---- error_from_sum / input_grad (no reference counterpart; the same batch checks) ---------------
def test_error_from_sum_and_input_grad_reject(ctx):
    db = block(ctx)
    s = torch.randn((65, 48), device="cuda")
    dx = torch.full((65, 32), 7.0, device="cuda")
    before = snap(db)
    assert st("skl_dense_error_from_sum", ctx.h, C.byref(db.desc()), C.c_void_p(s.data_ptr()), 65) == ALLOC_LIMIT
    assert st("skl_dense_error_from_sum", ctx.h, C.byref(db.desc()), C.c_void_p(s.data_ptr()), 0) == BAD_BATCH
    assert st("skl_dense_error_from_sum", ctx.h, C.byref(db.desc()), None, 64) == NULL_POINTER
    assert st("skl_dense_input_grad", ctx.h, C.byref(db.desc()), 65, C.c_void_p(dx.data_ptr())) == ALLOC_LIMIT
    assert st("skl_dense_input_grad", ctx.h, C.byref(db.desc()), 0, C.c_void_p(dx.data_ptr())) == BAD_BATCH
    assert_untouched(before, db)
    assert torch.all(dx == 7.0)


# ---- context, fill, cast ---------------------------------------------------------------------------
def test_context_and_fill_reject(ctx):
    h = C.c_void_p()
    assert abi.status("skl_ctx_create", 1 << 20, 16, C.byref(h)) == NO_DEVICE
    assert abi.status("skl_ctx_create", 0, 0, C.byref(h)) == INVALID_CONFIG
    buf = torch.full((16,), 3.0, device="cuda")
    assert st("skl_fill", ctx.h, C.c_void_p(buf.data_ptr()), 2, 1.0, 16) == INVALID_CONFIG
    assert torch.all(buf == 3.0)


@pytest.mark.parametrize("sdt,ddt", [(abi.F32, abi.F32), (abi.F16, abi.F16), (2, abi.F16), (abi.F32, 2)])
def test_cast_rejects_unsupported_pairs(ctx, sdt, ddt):
    """gpu_cast_t (util_device.rs:23-32) only knows f32 -> f16 and f16 -> f32."""
    src = torch.randn(64, device="cuda")
    dst = torch.full((64,), 5.0, device="cuda")
    assert st("skl_cast", ctx.h, C.c_void_p(src.data_ptr()), sdt, C.c_void_p(dst.data_ptr()), ddt, 32) \
        == UNSUPPORTED_CAST
    assert torch.all(dst == 5.0)


def _cast(ctx, src: torch.Tensor, sdt, ddt, out_dtype) -> torch.Tensor:
    dst = torch.empty(src.numel(), device="cuda", dtype=out_dtype)
    abi.call("skl_cast", ctx.h, C.c_void_p(src.data_ptr()), sdt, C.c_void_p(dst.data_ptr()), ddt, src.numel())
    torch.cuda.synchronize()
    return dst


def test_cast_f32_to_f16_round_to_nearest_even(ctx):
    """cast_f32_f16_t (util.cuh:9-13): IEEE round to nearest, ties to even, overflow to inf,
    gradual underflow; checked bit for bit against numpy's float32 -> float16."""
    g = rng(401)
    # every f16 exponent range, both signs
    mags = np.exp2(g.uniform(-27, 17, 200_000)).astype(np.float32)
    rand = mags * np.where(g.random(mags.size) < 0.5, -1, 1).astype(np.float32)
    # exact midpoints between adjacent finite f16 values (the ties), and their neighbours
    h = g.integers(0, 0x7BFF, 50_000).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float32)
    hi = (h + 1).view(np.float16).astype(np.float32)
    mid = ((lo.astype(np.float64) + hi) / 2).astype(np.float32)
    ties = np.concatenate([mid, -mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))])
    special = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.99, 65520.0, -65520.0, 1e30, -1e30,
                        2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, 6.097555e-05, 6.1035156e-05,
                        1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32)
    v = np.concatenate([rand, ties, special])
    got = _cast(ctx, torch.from_numpy(v).cuda(), abi.F32, abi.F16, torch.float16).cpu().numpy()
    want = v.astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    nan = np.array([np.nan, -np.nan], np.float32)
    assert np.all(np.isnan(_cast(ctx, torch.from_numpy(nan).cuda(), abi.F32, abi.F16, torch.float16).cpu().numpy()))


def test_cast_f16_to_f32_exact(ctx):
    """cast_f16_f32_t (util.cuh:15-19): every one of the 65536 f16 bit patterns widens exactly."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    v = bits.view(np.float16)
    got = _cast(ctx, torch.from_numpy(v.copy()).cuda(), abi.F16, abi.F32, torch.float32).cpu().numpy()
    want = v.astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
