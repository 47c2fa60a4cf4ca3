"""Pins of the CPU oracle (CPU only).

The reference ships no golden vectors or known-answer tests for this path
(its only test, src/lib.rs:56-137, runs one step on all-zero data and checks
nothing), so every oracle function is pinned here against what the
mathematics fixes: numpy's IEEE float16 conversion, numpy float64 matmul and
brute force, float64 closed forms and finite differences, invariants
(softmax rows sum to 1, dropout keep rate, idempotent rounding), Python
big-integer evaluation of the integer hashes, and hand-computed numbers for
the element-local norm gradient (util.cu:175-215), which deliberately differs
from autograd and is pinned by no other source.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import he_normal, rng

M32 = 0xFFFFFFFF


def rel(a, r):
    a, r = np.asarray(a, np.float64), np.asarray(r, np.float64)
    return float(np.max(np.abs(a - r)) / max(np.max(np.abs(r)), 1e-30))


# ---- binary16 ---------------------------------------------------------------------------------
def test_f16_rounding_matches_numpy_everywhere():
    g = rng(0)
    bits = g.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).astype(np.float32)
    got = O.round_f16(x)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("v", [0.0, -0.0, 1.0, 65504.0, 65520.0, 65519.99, 6.1035156e-05, 5.9604645e-08,
                               2.9802322e-08, 2.9802326e-08, 1.0009765625, 1.00048828125, 1.00146484375,
                               np.inf, -np.inf])
def test_f16_special_values(v):
    ref = np.float32(v).astype(np.float16).astype(np.float32)
    got = O.round_f16(np.array([v], np.float32))[0]
    assert np.float32(got).view(np.uint32) == np.float32(ref).view(np.uint32)


def test_f16_nan_and_idempotence():
    assert np.isnan(O.round_f16(np.array([np.nan], np.float32))[0])
    x = rng(1).standard_normal(10000).astype(np.float32) * 100
    once = O.round_f16(x)
    assert np.array_equal(O.round_f16(once), once)


# ---- integer hashes -----------------------------------------------------------------------------
def scramble_bigint(step, lid):
    h = (step * 1103515245 + lid) & M32
    h = ((h ^ (h >> 16)) * 1103515245) & M32
    return h ^ (h >> 15)


def dropout_bigint(col, row, seed):
    # math.cuh:45-53 with C's promotions spelled out: the col product is 64-bit.
    state = (((row * 1103515245) & M32) ^ ((col * 6364136223846793005) & 0xFFFFFFFFFFFFFFFF) ^ seed) & M32
    state ^= state >> 17
    state = (state * 1103515245 + 12345) & M32
    state ^= state >> 15
    return float(np.float32(state) / np.float32(4294967296.0))


def test_scramble_seed_bigint():
    g = rng(2)
    for _ in range(2000):
        s, i = int(g.integers(0, 2**32)), int(g.integers(0, 2**32))
        assert O.scramble_seed(s, i) == scramble_bigint(s, i)


def test_dropout_hash_bigint_and_truncated_constant():
    # the device code uses col * 0x4C957F2D: the low 32 bits of the 64-bit constant
    assert 6364136223846793005 & M32 == 0x4C957F2D
    g = rng(3)
    for _ in range(3000):
        c, r, s = (int(v) for v in g.integers(0, 2**32, 3))
        assert O.dropout_u(c, r, s) == dropout_bigint(c, r, s)


def test_dropout_uniformity_invariants():
    seed = O.scramble_seed(5, 27)
    u = np.array([O.dropout_u(c, r, seed + r * 7) for r in range(200) for c in range(250)])
    assert u.min() >= 0.0 and u.max() <= 1.0
    assert abs(np.mean(u >= 0.1) - 0.9) < 0.01
    assert abs(np.mean(u) - 0.5) < 0.01


# ---- activations ---------------------------------------------------------------------------------
def act64(act, x, leaky=0.01):
    x = np.float64(x)
    sig = 1 / (1 + np.exp(-x))
    return {0: x, 1: sig, 2: max(0.0, x), 3: x if x > 0 else leaky * x, 4: np.tanh(x), 5: x,
            6: x * sig, 7: x * np.tanh(np.log1p(np.exp(x)))}[act]


XS = np.concatenate([np.linspace(-15, 15, 301), [-0.5, 1e-3, 19.9, 20.1, 25.0]])


@pytest.mark.parametrize("act", range(8))
def test_activation_closed_forms(act):
    for x in XS:
        got = O.activation(act, float(x), 0.01)
        ref = act64(act, x)
        assert abs(got - ref) <= 2e-6 * max(1.0, abs(ref)), (act, x, got, ref)


@pytest.mark.parametrize("act", [1, 4, 6, 7])
def test_smooth_derivatives_match_finite_differences(act):
    h = 1e-5
    for x in np.linspace(-8, 8, 97):
        fd = (act64(act, x + h) - act64(act, x - h)) / (2 * h)
        out_v = O.activation(act, float(x), 0.0)
        got = O.activation_derivative(act, 1.0, out_v, float(x), 0.0)
        assert abs(got - fd) <= 2e-5 * max(1.0, abs(fd)), (act, x, got, fd)
        assert O.activation_derivative(act, -3.0, out_v, float(x), 0.0) == pytest.approx(-3.0 * got, rel=1e-6)


def test_relu_family_derivatives_use_post_activation_value():
    assert O.activation_derivative(2, 5.0, 0.3, -1.0, 0.0) == 5.0      # out_v > 0 decides, not in_x
    assert O.activation_derivative(2, 5.0, 0.0, 1.0, 0.0) == 0.0
    assert O.activation_derivative(3, 5.0, -0.1, 1.0, 0.01) == pytest.approx(0.05)
    assert O.activation_derivative(0, 5.0, 9.0, 9.0, 0.0) == 5.0
    assert O.activation_derivative(5, 5.0, 9.0, 9.0, 0.0) == 5.0


# ---- GEMM ----------------------------------------------------------------------------------------
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 7, 3), (17, 33, 19), (4, 1, 6), (64, 300, 48)])
def test_gemm_brute_force_and_numpy(m, k, n):
    g = rng(m * 100 + k)
    a = g.standard_normal((m, k)).astype(np.float32)
    b = g.standard_normal((k, n)).astype(np.float32)
    c = O.gemm_nn(a, b)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel(c, ref) < 1e-5
    if m * k * n <= 20000:
        for i in range(m):
            for j in range(n):
                s = sum(float(a[i, t]) * float(b[t, j]) for t in range(k))
                assert abs(c[i, j] - s) <= 1e-5 * (1 + abs(s))


# ---- forward ---------------------------------------------------------------------------------------
def fwd_pair(M, K, N, seed, **kw):
    g = rng(seed)
    w = he_normal(g, K, N)
    b = (g.standard_normal((1, N)) * 0.1).astype(np.float32)
    ob = O.OracleBlock(K, N, M, w, b=b, **kw)
    x = g.standard_normal((M, K)).astype(np.float32)
    return ob, x, w.astype(np.float64), b.astype(np.float64), x.astype(np.float64)


def test_forward_linear_relu_closed_form():
    ob, x, w, b, x64 = fwd_pair(40, 30, 20, 1, act=2)
    ob.forward(x, 40)
    z = x64 @ w + b
    assert rel(ob.preact, z) < 1e-5
    assert rel(ob.out, np.maximum(z, 0)) < 1e-5
    assert np.array_equal(ob.mask, np.ones_like(ob.mask))   # mask untouched without dropout


def test_forward_rmsnorm_closed_form():
    ob, x, w, b, x64 = fwd_pair(24, 16, 12, 2, norm=1, act=0)
    ob.norm_w[:] = rng(9).random((1, 12)).astype(np.float32) + 0.5
    ob.forward(x, 24)
    z = x64 @ w + b
    rstd = 1 / np.sqrt(np.mean(z * z, axis=1, keepdims=True) + 1e-6)
    assert rel(ob.prenorm, z) < 1e-5
    assert rel(ob.centered, z) < 1e-5
    assert rel(ob.norm_rstd[:24], rstd[:, 0]) < 1e-5
    assert rel(ob.preact, z * rstd * ob.norm_w.astype(np.float64)) < 1e-5


@pytest.mark.parametrize("norm", [2, 3])
def test_forward_layer_and_batch_norm_closed_form(norm):
    ob, x, w, b, x64 = fwd_pair(32, 16, 12, 3, norm=norm, act=4)
    g = rng(10)
    ob.norm_w[:] = g.random((1, 12)).astype(np.float32) + 0.5
    ob.norm_b[:] = g.standard_normal((1, 12)).astype(np.float32)
    ob.forward(x, 32)
    z = x64 @ w + (b if norm == 2 else 0)       # BatchNorm drops the linear bias
    ax = 1 if norm == 2 else 0
    mu = z.mean(axis=ax, keepdims=True)
    var = ((z - mu) ** 2).mean(axis=ax, keepdims=True)
    pre = (z - mu) / np.sqrt(var + 1e-6) * ob.norm_w + ob.norm_b
    assert rel(ob.centered, z - mu) < 1e-5
    assert rel(ob.preact, pre) < 1e-5
    assert rel(ob.out, np.tanh(pre)) < 1e-5
    rows = 32 if norm == 2 else 12
    assert rel(ob.norm_rstd[:rows], (1 / np.sqrt(var + 1e-6)).ravel()) < 1e-5


def test_forward_dropout_invariants():
    ob, x, *_ = fwd_pair(200, 20, 100, 4, act=6, mask_coeff=0.25)
    ob.forward(x, 200, True, O.scramble_seed(9, 44))
    keep = ob.mask > 0
    assert set(np.unique(ob.mask)) <= {0.0, np.float32(1 / 0.75)}
    assert abs(keep.mean() - 0.75) < 0.02
    assert np.allclose(ob.out, ob.predrop * ob.mask, rtol=1e-6, atol=0)


def test_forward_half_mode_stores_f16_values():
    ob, x, *_ = fwd_pair(16, 8, 8, 5, half=True, norm=1, act=7, mask_coeff=0.1)
    ob.forward(O.round_f16(x), 16, True, 77)
    for n in ("prenorm", "preact", "predrop", "out", "mask", "centered"):
        a = getattr(ob, n)
        assert np.array_equal(O.round_f16(a), a), n


# ---- softmax / loss delta -------------------------------------------------------------------------
def out_pair(M, N, seed, loss, act, norm=0):
    ob, x, w, b, x64 = fwd_pair(M, 8, N, seed, act=0, norm=norm)
    ob.forward(x, M)
    z = x64 @ w + b
    g = rng(seed + 50)
    t = np.zeros((M, N), np.float32)
    t[np.arange(M), g.integers(0, N, M)] = 1
    ob.output_error(t, loss, act)
    return ob, z, t.astype(np.float64)


def test_softmax_ce_delta():
    ob, z, t = out_pair(20, 10, 6, 1, 5)
    p = np.exp(z - z.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    assert rel(ob.out, p) < 1e-5
    assert np.allclose(ob.out.sum(1), 1.0, atol=1e-6)
    assert rel(ob.grad, p - t) < 1e-5
    assert rel(ob.d_prenorm, 512 * (p - t)) < 1e-5      # LOSS_SCALE on the output layer
    assert not ob.d_norm_w.any() and not ob.d_norm_b.any()


def test_bce_and_mse_deltas():
    ob, z, t = out_pair(20, 6, 7, 2, 1)
    s = 1 / (1 + np.exp(-z))
    assert rel(ob.grad, s - t) < 1e-5
    ob, z, t = out_pair(20, 6, 8, 0, 0)
    assert rel(ob.grad, z - t) < 1e-5
    ob, z, t = out_pair(20, 6, 9, 0, 1)
    s = 1 / (1 + np.exp(-z))
    assert rel(ob.grad, (s - t) * s * (1 - s)) < 1e-5


def test_bad_pairing_gives_zero_delta():
    # CE without Softmax falls through to err = 0 (backward.cu:31-43); the C ABI rejects the pairing first
    ob, z, t = out_pair(8, 4, 10, 1, 0)
    assert not ob.grad.any()


# ---- element-local norm gradient: hand-computed numbers ---------------------------------------------
def _one_row_block(norm, p, c, rstd, nw):
    ob = O.OracleBlock(1, 4, 1, np.zeros((1, 4), np.float32), norm=norm, act=0)
    ob.prenorm[:] = p
    ob.centered[:] = c
    ob.norm_rstd[:] = rstd
    ob.norm_w[:] = nw
    ob.out[:] = 1.0            # MSE with identity: e = out - target = 1
    ob.preact[:] = 1.0
    ob.output_error(np.zeros((1, 4), np.float32), 0, 0)
    return ob


def test_rms_norm_gradient_hand_values():
    # e = 1, p = 2, rstd = 0.5, N = 4, g = 1:
    #   dNw = e p rstd = 1;  d = g rstd (e - rstd^2 p^2 / N) = 0.5 * (1 - 0.25) = 0.375;  x512 = 192
    ob = _one_row_block(1, 2.0, 0.0, 0.5, 1.0)
    assert np.allclose(ob.d_norm_w, 1.0) and np.allclose(ob.d_norm_b, 0.0)
    assert np.allclose(ob.d_prenorm, 192.0)
    # g = 2 doubles d: 384
    ob = _one_row_block(1, 2.0, 0.0, 0.5, 2.0)
    assert np.allclose(ob.d_prenorm, 384.0)


def test_layer_norm_gradient_hand_values():
    # e = 1, c = 2, rstd = 0.5, N = 4: d = 0.5 (1 - 1/4 - 0.25 * 4 * 1/4) = 0.25 -> x512 = 128;
    # dNw = e c rstd = 1; dNb = e = 1
    ob = _one_row_block(2, 0.0, 2.0, 0.5, 1.0)
    assert np.allclose(ob.d_prenorm, 128.0)
    assert np.allclose(ob.d_norm_w, 1.0) and np.allclose(ob.d_norm_b, 1.0)


def test_batch_norm_gradient_hand_values():
    # m = 1 row: d = 0.5 (1 - 1/1 - 0.25 * 4 * 1/1) = -0.5 -> x512 = -256
    ob = _one_row_block(3, 0.0, 2.0, 0.5, 1.0)
    assert np.allclose(ob.d_prenorm, -256.0)


def _norm_grad_block(norm, e, M=2, N=4, p=2.0, c=2.0, rstd=0.5, nw=1.5):
    """M x N output block whose error is e everywhere (MSE + identity: e = out - target, target 0),
    prenorm p and centered c set apart so that a formula reading the wrong one fails."""
    ob = O.OracleBlock(1, N, M, np.zeros((1, N), np.float32), norm=norm, act=0)
    ob.prenorm[:] = p
    ob.centered[:] = c
    ob.norm_rstd[:] = rstd
    ob.norm_w[:] = nw
    ob.out[:] = e
    ob.preact[:] = 1.0
    ob.output_error(np.zeros((M, N), np.float32), 0, 0)
    return ob


# Hand values with e != 1 (util.cu:187-210, Q3).  With e = 1 the reference's
# missing e factor in the RMS second term, and the e factor of the LN / BN third
# term, cannot be seen; each case below names the value the "fixed" formula
# would give, which the oracle must NOT produce.  Common: g = 1.5, rstd = 0.5,
# N = 4; the output layer's d_prenorm carries LOSS_SCALE = 512, dNorm does not.
@pytest.mark.parametrize("e,d,d_fixed,dnw", [
    # RMS, p = 2 (c = 7 ignored): d = g r (e - r^2 p^2 / N) = 0.75 (e - 0.25)
    (2.0, 0.75 * 1.75, 0.75 * (2.0 - 0.5), 2.0),          # 672;  e r^2 p^2 / N would give 576
    (-0.5, 0.75 * -0.75, 0.75 * (-0.5 + 0.125), -0.5),    # -288; e r^2 p^2 / N would give -144
])
def test_rms_norm_gradient_hand_values_e_not_one(e, d, d_fixed, dnw):
    ob = _norm_grad_block(1, e, p=2.0, c=7.0)
    assert np.all(ob.d_prenorm == np.float32(512 * d))
    assert not np.any(ob.d_prenorm == np.float32(512 * d_fixed))
    assert np.all(ob.d_norm_w == np.float32(dnw))          # dNw = e p rstd
    assert not ob.d_norm_b.any()


@pytest.mark.parametrize("e,d,d_fixed,dnw", [
    # LN, c = 2 (p = 5 ignored): d = g r (e - e / N - r^2 c^2 e / N) = 0.75 (e - e/4 - e/4)
    (2.0, 0.75 * (2.0 - 0.5 - 0.5), 0.75 * (2.0 - 0.5 - 0.25), 2.0),          # 384; without e: 480
    (-0.5, 0.75 * (-0.5 + 0.125 + 0.125), 0.75 * (-0.5 + 0.125 - 0.25), -0.5),  # -96; without e: -240
])
def test_layer_norm_gradient_hand_values_e_not_one(e, d, d_fixed, dnw):
    ob = _norm_grad_block(2, e, p=5.0, c=2.0)
    assert np.all(ob.d_prenorm == np.float32(512 * d))
    assert not np.any(ob.d_prenorm == np.float32(512 * d_fixed))
    assert np.all(ob.d_norm_w == np.float32(dnw))          # dNw = e c rstd
    assert np.all(ob.d_norm_b == np.float32(e))            # dNb = e


@pytest.mark.parametrize("e,d,d_fixed,d_inv_n", [
    # BN over m = 2 rows, c = 1 (p = 5 ignored): d = g r (e - e / m - r^2 c^2 e / m) = 0.75 (e - e/2 - e/8)
    (2.0, 0.75 * (2.0 - 1.0 - 0.25), 0.75 * (2.0 - 1.0 - 0.125), 0.75 * (2.0 - 0.5 - 0.125)),
    (-0.5, 0.75 * (-0.5 + 0.25 + 0.0625), 0.75 * (-0.5 + 0.25 - 0.125), 0.75 * (-0.5 + 0.125 + 0.03125)),
])
def test_batch_norm_gradient_hand_values_e_not_one(e, d, d_fixed, d_inv_n):
    ob = _norm_grad_block(3, e, M=2, N=4, p=5.0, c=1.0)
    assert np.all(ob.d_prenorm == np.float32(512 * d))
    assert not np.any(ob.d_prenorm == np.float32(512 * d_fixed))     # third term without e
    assert not np.any(ob.d_prenorm == np.float32(512 * d_inv_n))     # 1/N (columns) instead of 1/m (rows)
    assert np.all(ob.d_norm_w == np.float32(e * 1.0 * 0.5))
    assert np.all(ob.d_norm_b == np.float32(e))


def test_rms_forward_fp16_rounds_twice():
    """forward.cu:61-72 with T = half: preact = T(T(prenorm * rstd) * norm_w), rstd = T(rsqrt(...)).
    One row of four f16 values (x = [1], W = that row), worked by hand in exact fractions:
    sum z^2 / 4 + 1e-6 -> rstd32 = 0.197476 -> T: 809/4096.  Element 0:
    z r = 837/128 * 809/4096 = 1322.52 / 1024 -> 1323/1024; * 351/512 = 1813.96 / 2048 -> 907/1024.
    One rounding of z r g = 1813.30 / 2048 would give 1813/2048 instead."""
    z = np.array([[837 / 128, 675 / 256, 927 / 256, 807 / 128]], np.float32)
    gw = np.array([[351 / 512, 977 / 1024, 703 / 1024, 151 / 128]], np.float32)
    ob = O.OracleBlock(1, 4, 1, z, half=True, norm=1, act=0)
    ob.norm_w[:] = gw
    ob.forward(np.ones((1, 1), np.float32), 1)
    assert ob.norm_rstd[0] == np.float32(809 / 4096)
    assert np.array_equal(ob.prenorm, z) and np.array_equal(ob.centered, z)
    twice = np.array([[907 / 1024, 509 / 1024, 503 / 1024, 47 / 32]], np.float32)
    once = np.array([[1813 / 2048, 2035 / 4096, 2011 / 4096, 47 / 32]], np.float32)
    assert np.array_equal(ob.preact, twice)
    assert np.sum(ob.preact != once) == 3
    # the fp32 block rounds nowhere: z * rstd32 * g in f32 (rstd not rounded to f16)
    o32 = O.OracleBlock(1, 4, 1, z, norm=1, act=0)
    o32.norm_w[:] = gw
    o32.forward(np.ones((1, 1), np.float32), 1)
    assert abs(o32.norm_rstd[0] - 0.197476) < 1e-6
    assert np.allclose(o32.preact, z * o32.norm_rstd[0] * gw, rtol=1e-6, atol=0)


# ---- hidden error / input gradient ---------------------------------------------------------------------
def test_hidden_error_and_input_grad_closed_form():
    M, K0, N0, N1 = 30, 12, 20, 7
    g = rng(11)
    o0 = O.OracleBlock(K0, N0, M, he_normal(g, K0, N0), act=2)
    o1 = O.OracleBlock(N0, N1, M, he_normal(g, N0, N1), act=0)
    x = g.standard_normal((M, K0)).astype(np.float32)
    o0.forward(x, M)
    o1.forward(o0.out, M)
    t = np.zeros((M, N1), np.float32)
    t[np.arange(M), g.integers(0, N1, M)] = 1
    o1.output_error(t, 1, 5)
    o0.hidden_error(o1, M)
    s = o1.d_prenorm.astype(np.float64) @ o1.w.astype(np.float64).T
    assert rel(o0.grad, s * (o0.predrop > 0)) < 1e-5
    assert rel(o1.input_grad(M), s) < 1e-5


def test_hidden_error_and_input_grad_fp16_operands_rounded():
    """backward_wmma.cu:44,51: in half mode the dX GEMM rounds both operands to f16 (d_prenorm and the
    next layer's fp32 master W) and accumulates in f32.  Every operand is 0.45 fp16 ulp above an fp16
    value in [1, 2), so each rounding moves it down by 0.45 ulp (2^-10): the oracle must agree with
    float64 on the rounded operands to f32 summation noise, and disagree with the product of the
    unrounded operands, or of either one unrounded, by far more than that."""
    M, K0, N0, N1 = 20, 8, 48, 64
    g = rng(31)

    def off_grid(shape):
        return (1.0 + (g.integers(0, 1000, shape) + 0.45) * 2.0 ** -10).astype(np.float32)

    wm = off_grid((N0, N1))
    o0 = O.OracleBlock(K0, N0, M, he_normal(g, K0, N0), half=True, act=0)
    o1 = O.OracleBlock(N0, N1, M, O.round_f16(wm), half=True, act=0, master_w=wm)
    s = off_grid((M, N1))
    o1.error_from_sum(s, M)                   # identity, no norm: d_prenorm = s
    assert np.array_equal(o1.d_prenorm, s)
    dp64, w64 = s.astype(np.float64), wm.astype(np.float64)
    rounded = O.round_f16(s).astype(np.float64) @ O.round_f16(wm).astype(np.float64).T
    scale = np.abs(O.round_f16(s)).astype(np.float64) @ np.abs(O.round_f16(wm)).astype(np.float64).T
    tol = 4 * N1 * 2.0 ** -24                  # sequential f32 accumulation of N1 terms
    dx = o1.input_grad(M)
    o0.hidden_error(o1, M)                    # identity: grad = mask * s = s
    for name, got in (("input_grad", dx), ("hidden_error grad", o0.grad[:M])):
        err = np.max(np.abs(got - rounded) / scale)
        miss = np.max(np.abs(dp64 @ w64.T - rounded) / scale)
        only_dp = np.max(np.abs(O.round_f16(s).astype(np.float64) @ w64.T - rounded) / scale)
        only_w = np.max(np.abs(dp64 @ O.round_f16(wm).astype(np.float64).T - rounded) / scale)
        assert err < tol, (name, err)
        assert min(miss, only_dp, only_w) > 10 * tol, (name, miss, only_dp, only_w)


# ---- optimisers --------------------------------------------------------------------------------------------
def bwd_setup(seed, M=48, K=16, N=12, **kw):
    g = rng(seed)
    w = he_normal(g, K, N)
    ob = O.OracleBlock(K, N, M, w, act=0, **kw)
    x = g.standard_normal((M, K)).astype(np.float32)
    dp = (g.standard_normal((M, N)) * 512).astype(np.float32)
    ob.d_prenorm[:] = dp
    gw = (x.astype(np.float64).T @ dp.astype(np.float64)) / 512 / M
    gb = dp.astype(np.float64).sum(0, keepdims=True) / 512 / M
    return ob, x, w.astype(np.float64), gw, gb


def test_sgd_closed_form():
    ob, x, w, gw, gb = bwd_setup(12)
    ob.backward(x, O.Optimiser.sgd(0.0), O.Optimiser.sgd(0.0), 48, 0.1, 3.4e38, 1)
    assert rel(ob.dv_w, gw) < 1e-5               # SGD momentum buffer holds the step gradient
    assert rel(ob.w, w - 0.1 * gw) < 1e-5
    assert rel(ob.b, -0.1 * gb) < 1e-5
    assert not ob.dm_w.any()


def test_sgd_nesterov_first_step():
    ob, x, w, gw, _ = bwd_setup(13)
    ob.backward(x, O.Optimiser.sgd(0.9, True), O.Optimiser.sgd(0.9, True), 48, 0.1, 3.4e38, 1)
    assert rel(ob.w, w - 0.1 * gw * 1.9) < 1e-5   # v = g; u = lr (g + 0.9 v)


def test_adam_first_step_closed_form():
    ob, x, w, gw, _ = bwd_setup(14)
    ob.backward(x, O.Optimiser.adam(0.9, 0.999, 1e-8), O.Optimiser.adam(), 48, 1e-3, 3.4e38, 1)
    c1 = float(np.float32(1.0) - np.float32(0.9))      # (1 - beta) as fp32 arithmetic forms it
    c2 = float(np.float32(1.0) - np.float32(0.999))
    assert rel(ob.dm_w, c1 * gw) < 1e-5
    assert rel(ob.dv_w, c2 * gw * gw) < 1e-5
    assert rel(ob.w - w, -1e-3 * gw / (np.abs(gw) + 1e-8)) < 1e-4


def test_clamp_applies_to_the_update():
    ob, x, w, gw, _ = bwd_setup(15)
    ob.backward(x, O.Optimiser.sgd(0.0), O.Optimiser.sgd(0.0), 48, 1.0, 1e-3, 1)
    assert rel(ob.w, w - np.clip(gw, -1e-3, 1e-3)) < 1e-5


@pytest.mark.parametrize("regu,c", [(1, 1e-3), (2, 1e-2)])
def test_regularisation_closed_form(regu, c):
    ob, x, w, gw, _ = bwd_setup(16, regularisation=regu, regu_coeff=c)
    ob.backward(x, O.Optimiser.sgd(0.0), O.Optimiser.sgd(0.0), 48, 0.1, 3.4e38, 1)
    pre = w - c * np.sign(w) if regu == 1 else w * (1 - 2 * c)
    assert rel(ob.w, pre - 0.1 * gw) < 1e-5


def test_norm_param_sums_and_half_master():
    ob, x, w, gw, gb = bwd_setup(17, half=True, norm=2)
    ob.d_norm_w[:] = rng(18).standard_normal(ob.d_norm_w.shape).astype(np.float32)
    ob.d_norm_b[:] = rng(19).standard_normal(ob.d_norm_b.shape).astype(np.float32)
    gnw = ob.d_norm_w.astype(np.float64).sum(0, keepdims=True) / 512 / 48
    ob.backward(O.round_f16(x), O.Optimiser.sgd(0.0), O.Optimiser.sgd(0.0), 48, 0.1, 3.4e38, 1)
    assert rel(ob.dv_norm_w, gnw) < 1e-5
    assert rel(ob.master_norm_w, 1 - 0.1 * gnw) < 1e-5
    assert np.array_equal(ob.norm_w, O.round_f16(ob.master_norm_w))
    assert np.array_equal(ob.w, O.round_f16(ob.master_w))


# ---- network order: update before propagate (src/ffn.rs:142-163) -------------------------------------------
def test_hidden_error_uses_updated_next_layer():
    M = 16
    g = rng(20)
    o0 = O.OracleBlock(6, 5, M, he_normal(g, 6, 5), act=6)
    o1 = O.OracleBlock(5, 3, M, he_normal(g, 5, 3), act=0)
    x = g.standard_normal((M, 6)).astype(np.float32)
    o0.forward(x, M)
    h = o0.out.copy()
    o1.forward(h, M)
    t = np.zeros((M, 3), np.float32)
    t[np.arange(M), g.integers(0, 3, M)] = 1
    o1.output_error(t, 1, 5)
    w1_old = o1.w.astype(np.float64).copy()
    o1.backward(h, O.Optimiser.sgd(0.0), O.Optimiser.sgd(0.0), M, 0.5, 3.4e38, 1)
    o0.hidden_error(o1, M)
    s_new = o1.d_prenorm.astype(np.float64) @ o1.w.astype(np.float64).T
    s_old = o1.d_prenorm.astype(np.float64) @ w1_old.T
    d = np.array([[O.activation_derivative(6, 1.0, float(o0.predrop[i, j]), float(o0.preact[i, j]), 0)
                   for j in range(5)] for i in range(M)])
    assert rel(o0.grad, s_new * d) < 1e-5
    assert rel(o0.grad, s_old * d) > 1e-3


def test_reference_order_fp32_noise_exceeds_elementwise_1e4():
    """The reference sums its fp32 GEMMs sequentially over k (math.cu:8-50, backward.cu:181-186); the
    oracle does the same.  Against exact (float64) arithmetic that order is already further than 1e-4
    away in the elementwise metric (near-zero outputs of long sums), while it is ~1e-6 normwise: the
    parity gates therefore bound fp32 elementwise errors at 1e-2, not 1e-4 (tests/helpers.py)."""
    from tests.helpers import elementwise, normwise
    M, K, N = 1024, 1024, 256
    g = rng(77)
    w = he_normal(g, K, N)
    x = g.standard_normal((M, K)).astype(np.float32)
    ob = O.OracleBlock(K, N, M, w, act=0)
    ob.forward(x, M)
    exact = x.astype(np.float64) @ w.astype(np.float64)
    ew, nw = elementwise(ob.preact, exact), normwise(ob.preact, exact)
    assert 1e-4 < ew < 1e-2, ew
    assert nw < 1e-5, nw
