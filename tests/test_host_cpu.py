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
