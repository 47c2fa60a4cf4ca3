"""The C++ host API (soklyn_amd/host) on the CPU: its self-test, and the initialiser
stack of src/util/function.rs:190-319 pinned piece by piece.

- ChaCha block function: against OpenSSL's RFC 7539 ChaCha20 keystream
  (tests/golden/chacha20_keystream.txt, made by tests/golden/make_chacha20_vectors.sh;
  the all-zero-key line is RFC 7539 appendix A.1 test vector 1).  ChaCha8 is the same
  function with 8 rounds.
- PCG32 (rand_core's seed_from_u64 expansion): XSH-RR output and LCG multiplier against
  pcg-c's published pcg32-demo sequence for seed 42, sequence 54.
- Box-Muller / uniform mappings: distribution checks (moments, Kolmogorov-Smirnov),
  exact scaling by the power-of-two factor, determinism per seed.
Parity unpinned: the bitwise values of the reference's InitFuncs (rand_core's PCG
increment and advance-before-output order, and Rust's f32 ln/cos ulps) - no vector of
the reference's own output exists to check them against.
"""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest
from scipy import stats

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "soklyn_amd", "host", "soklyn_tool")
GOLDEN = os.path.join(ROOT, "tests", "golden", "chacha20_keystream.txt")


def tool(*args) -> str:
    if not os.path.exists(TOOL):
        pytest.fail("soklyn_tool is not built (run __graft_entry__.build())")
    p = subprocess.run([TOOL, *map(str, args)], capture_output=True, text=True, timeout=120)
    assert p.returncode == 0, p.stdout + p.stderr
    return p.stdout


def init_values(kind, seed, factor, fan_in, fan_out, n) -> np.ndarray:
    words = tool("init", kind, seed, factor, fan_in, fan_out, n).split()
    return np.array([int(w, 16) for w in words], dtype=np.uint32).view(np.float32)


def test_selftest():
    assert tool("selftest").strip() == "OK"


def test_chacha20_block_matches_openssl():
    lines = open(GOLDEN).read().split("\n")
    assert len([l for l in lines if l.strip()]) == 3
    for line in lines:
        if not line.strip():
            continue
        key, ctr, n, *words = line.split()
        got = tool("chacha", 20, key, ctr, n).split()
        assert got == words, key


def test_rfc7539_zero_key_vector():
    # RFC 7539 A.1 test vector 1 begins 76 b8 e0 ad a0 f1 3d 90 (little-endian word ade0b876)
    assert tool("chacha", 20, "0" * 64, 0, 1).split()[:2] == ["ade0b876", "903df1a0"]


def test_chacha8_differs_from_chacha20_and_is_deterministic():
    k = "000102030405060708090a0b0c0d0e0f101112131415161718191a1b1c1d1e1f"
    a, b = tool("chacha", 8, k, 0, 2), tool("chacha", 8, k, 0, 2)
    assert a == b and a != tool("chacha", 20, k, 0, 2)


def test_pcg32_demo_sequence():
    assert tool("pcg32", 42, 54, 6).split() == ["a15c02b7", "7b47f409", "ba1d3330", "83d2f293", "bfa4784b",
                                                "cbed606e"]


@pytest.mark.parametrize("kind,fan_in,fan_out,std", [
    ("he_normal", 256, 64, np.sqrt(2.0 / 256)),
    ("xavier_normal", 300, 100, np.sqrt(2.0 / 400)),
])
def test_normal_initialisers(kind, fan_in, fan_out, std):
    n = 100_000
    v = init_values(kind, 7, 1.0, fan_in, fan_out, n).astype(np.float64)
    assert abs(v.mean()) < 5 * std / np.sqrt(n)
    assert abs(v.std() / std - 1) < 0.01
    assert stats.kstest(v / std, "norm").pvalue > 1e-3


@pytest.mark.parametrize("kind,fan_in,fan_out,limit", [
    ("he_uniform", 256, 64, np.sqrt(6.0 / 256)),
    ("xavier_uniform", 300, 100, np.sqrt(6.0 / 400)),
])
def test_uniform_initialisers(kind, fan_in, fan_out, limit):
    n = 100_000
    v = init_values(kind, 11, 1.0, fan_in, fan_out, n).astype(np.float64)
    assert v.min() >= -limit * (1 + 1e-6) and v.max() <= limit * (1 + 1e-6)
    assert stats.kstest((v + limit) / (2 * limit), "uniform").pvalue > 1e-3


def test_initialiser_factor_seed_and_determinism():
    a = init_values("he_normal", 3, 1.0, 64, 32, 512)
    assert np.array_equal(a, init_values("he_normal", 3, 1.0, 64, 32, 512))
    assert not np.array_equal(a, init_values("he_normal", 4, 1.0, 64, 32, 512))
    # T::from_f32(factor * z * std): a power-of-two factor scales every value exactly
    assert np.array_equal(init_values("he_normal", 3, 0.5, 64, 32, 512), a * np.float32(0.5))


# ---- learning-rate schedulers (src/util/scheduler.rs) ----------------------------------------------
def sched(*args):
    lines = tool("sched", *args).strip().splitlines()
    seq = np.array([int(w, 16) for w in lines[0].split()], np.uint32).view(np.float32)
    reset = (np.array([int(lines[1].split()[1], 16)], np.uint32).view(np.float32)[0] if len(lines) > 1 else None)
    return seq, reset


def test_cosine_decay_lr_closed_form():
    """scheduler.rs:38-57: linear warm-up min -> max over W steps, then min + (max - min)/2 (1 + cos(pi p))
    with p = (step - W) / (T - W); the endpoints are exact, no clamp past T, reset returns to step 0."""
    lo, hi, T, W = 1e-4, 3e-3, 20, 5
    seq, reset = sched("cosine", lo, hi, T, W, T + 4)
    lo32, hi32 = np.float32(lo), np.float32(hi)
    # warm-up: f32 arithmetic of the reference, exactly
    for s in range(W):
        p = np.float32(s) / np.float32(W)
        assert seq[s] == lo32 + p * (hi32 - lo32), s
    assert seq[W] == hi32                      # cos(0) = 1: the peak, exactly
    assert seq[T] == lo32                      # cos(pi) = -1 in f32: the floor, exactly
    mid = W + (T - W) // 2 if (T - W) % 2 == 0 else None
    steps = np.arange(T + 5, dtype=np.float64)
    p = (steps - W) / (T - W)
    ref = lo + 0.5 * (hi - lo) * (1 + np.cos(np.pi * p))
    dec = steps >= W
    assert np.allclose(seq[dec], ref[dec], rtol=2e-6, atol=0)
    assert np.all(np.diff(seq[W:T + 1]) < 0)   # strictly decreasing over the decay
    assert np.all(np.diff(seq[T:]) > 0)        # and back up past T (the cosine is not clamped)
    assert reset == seq[0] == lo32
    if mid is not None:
        assert abs(seq[mid] - (lo + hi) / 2) < 1e-7


def test_cosine_decay_lr_degenerate_decay():
    seq, _ = sched("cosine", 0.5, 1.0, 4, 4, 6)   # T == W: the rate drops to min after the warm-up
    assert np.array_equal(seq[:4], np.float32([0.5, 0.625, 0.75, 0.875]))
    assert np.all(seq[4:] == np.float32(0.5))
    seq, _ = sched("cosine", 0.5, 1.0, 6, 0, 2)   # no warm-up: starts at the peak
    assert seq[0] == np.float32(1.0)


def test_exponential_lr_sequence():
    """scheduler.rs:115-119: cur *= factor, in f32, each step; reset restores the initial rate."""
    seq, reset = sched("exp", 0.1, 0.7, 30)
    want = [np.float32(0.1)]
    for _ in range(30):
        want.append(np.float32(want[-1] * np.float32(0.7)))
    assert np.array_equal(seq, np.array(want, np.float32))
    assert reset == np.float32(0.1)
    assert np.allclose(seq, 0.1 * 0.7 ** np.arange(31), rtol=1e-5, atol=0)


def _plateau_model(patience, maximize, factor, min_lr, reset_lr, vals):
    """The same state machine, written from its specification (scheduler.rs:196-231)."""
    best = -np.inf if maximize else np.inf
    lr, t, out = np.float32(reset_lr), 0, []
    for v in vals:
        if not np.isnan(v):
            if (v > best) if maximize else (v < best):
                best, t = v, 0
            else:
                t += 1
                if t == patience:
                    t, lr = 0, max(np.float32(lr * np.float32(factor)), np.float32(min_lr))
        out.append(lr)
    return np.array(out, np.float32)


@pytest.mark.parametrize("mode", ["min", "max"])
def test_reduce_lr_on_plateau_patience_and_floor(mode):
    """Patience counts consecutive non-improving steps (equal values do not improve), the count restarts
    after each reduction and after each improvement, NaN steps change nothing, and the rate stops at
    min_lr; before reset() the rate is 0, as in the reference."""
    sign = 1.0 if mode == "min" else -1.0
    vals = sign * np.array([1.0, 0.9, 0.9, 0.95, np.nan, 0.8, 1, 1, 1, 1, 1, 1, 1, 0.5, 0.7, 0.7, 0.7], np.float32)
    seq, _ = sched("plateau", 2, mode, 0.5, 0.01, 0.1, *[f"{v:.9g}" for v in vals])
    assert seq[0] == 0.0 and seq[1] == np.float32(0.1)
    got = seq[2:]
    want = _plateau_model(2, mode == "max", 0.5, 0.01, 0.1, vals)
    assert np.array_equal(got, want)
    # hand values: reductions after the 2nd non-improving step, floored at 0.01
    assert np.array_equal(got[:13], np.float32([0.1, 0.1, 0.1, 0.05, 0.05, 0.05, 0.05, 0.025, 0.025, 0.0125,
                                                0.0125, 0.01, 0.01]))


def test_reduce_lr_on_plateau_zero_patience_fails():
    p = subprocess.run([TOOL, "sched", "plateau", "0", "min", "0.5", "0.01", "0.1"], capture_output=True, text=True)
    assert p.returncode != 0 and "Patience must be non-zero" in p.stderr
