"""The oracle against the repository's committed golden vectors (tests/golden/oracle_tiny.npz,
from tests/golden/make_oracle_vectors.py): re-running the tiny cases must reproduce every
committed input and output bit for bit, so any change to the oracle's arithmetic shows up
here before it can move the GPU parity gates."""
from __future__ import annotations

import os

import numpy as np
import pytest

from tests.golden import cases
from tests.golden.make_oracle_vectors import oracle_case

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_tiny.npz")


@pytest.fixture(scope="module")
def golden():
    with np.load(FIXTURE, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", list(cases.CASES))
def test_oracle_reproduces_golden_vectors(golden, name):
    d = cases.inputs(name)
    for k, v in d.items():
        assert np.array_equal(golden[f"{name}__in__{k}"], v), f"input {k}"
    res = oracle_case(name, d)
    keys = [k for k in golden if k.startswith(f"{name}__out__")]
    assert len(keys) == len(res)
    for k, v in res.items():
        ref = golden[f"{name}__out__{k}"]
        assert np.array_equal(ref, v, equal_nan=True), f"{name} {k}: max |diff| {np.nanmax(np.abs(ref - v)):.3e}"
