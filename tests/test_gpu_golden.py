"""The device against the committed golden vectors (tests/golden/oracle_tiny.npz): the tiny
cases of tests/golden/cases.py run through the C ABI on the committed inputs; gates
fp32 1e-4 normwise and 1e-2 elementwise, fp16 2e-2 normwise, dropout masks bit-exact."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from soklyn_amd import abi
from soklyn_amd.devblock import DeviceBlock
from tests.golden import cases
from tests.helpers import FP16_TOL, FP32_TOL, check

pytestmark = pytest.mark.gpu

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "oracle_tiny.npz")


@pytest.mark.parametrize("name", list(cases.CASES))
def test_device_matches_golden_vectors(ctx, name):
    with np.load(FIXTURE, allow_pickle=False) as z:
        g = {k: z[k] for k in z.files}
    d = {k[len(name) + 6:]: v for k, v in g.items() if k.startswith(f"{name}__in__")}

    def make(K, N, M, w, half, b, **kw):
        return DeviceBlock(ctx, K, N, M, w, half=half, master_w=w if half else None, b=b, **kw)

    def opt(spec):
        return abi.adam() if spec[0] == "adam" else abi.sgd(spec[1], spec[2])

    def to_dev(a, half):
        t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
        return t.half() if half else t

    res = cases.run(name, d, make, opt, lambda o, M, lr: (abi.train_ctx(o, o, M, lr), 1), to_dev,
                    lambda t: t.float().cpu().numpy())
    torch.cuda.synchronize()
    tol = FP16_TOL if cases.CASES[name]["half"] else FP32_TOL
    for k, v in res.items():
        ref = g[f"{name}__out__{k}"]
        if k.startswith("mask"):
            assert np.array_equal(v, ref), f"{name} {k}"
        else:
            check(f"{name} {k}", v, ref, tol)
