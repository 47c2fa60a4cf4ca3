"""fp16 blocks whose d_prenorm leaves the fp16 range.

The device feeds its dW and dX GEMMs the fp16 copy d_prenorm_h.  The reference
rounds d_prenorm to fp16 only for its dX (backward_wmma.cu:44) and sums its dW
in fp32 from the fp32 d_prenorm (backward.cu:181-186), so where |d_prenorm| >
65504 its dW stays finite while an fp16 copy of those values is infinite.  The
device sums such elements again in fp32 from d_prenorm (in the optimiser
epilogue of every dW path: the fused direct-to-LDS and register-staged kernels,
the padded element-wise epilogue, the split-K reduction), so W, its master and
both moments must come out finite and match the oracle, whose dW is the
reference's fp32 sum.  The dX of such a block is infinite on both sides (the
reference rounds dX's operand to fp16 as well).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soklyn_amd import abi
from tests.helpers import FP16_TOL, check, rng
from tests.test_gpu_parity import dev, inputs, make_pair

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,K,N,what", [
    (512, 4096, 3072, "direct-to-LDS dW + Adam, whole tiles, no split-K"),
    (6000, 1000, 1531, "direct-to-LDS split-K partials on zero-padded operands + reduction"),
    (300, 4000, 3001, "zero-padded operands: element-wise Adam epilogue"),
    (256, 128, 160, "register-staged dW + Adam"),
    (4096, 512, 512, "register-staged split-K partials + reduction"),
])
def test_dw_finite_where_d_prenorm_saturates_fp16(ctx, M, K, N, what):
    print(f"[case] {what}: M={M} K={K} N={N}", flush=True)
    ob, db = make_pair(ctx, K, N, M, seed=M + K + N, half=True, act=abi.ACT_IDENTITY)
    x = inputs(K + 1, M, K, True)
    ob.forward(x, M)
    db.forward(dev(x, True), M)
    g = rng(N + 2)
    s = (g.standard_normal((M, N)) * 512).astype(np.float32)
    cols = g.choice(N, size=max(1, N // 64), replace=False)
    s[:, cols] *= 400.0                     # |d_prenorm| up to ~1e6 in these columns: fp16 overflows
    ob.error_from_sum(s, M)
    db.error_from_sum(torch.from_numpy(s).cuda(), M)
    torch.cuda.synchronize()
    h = db.d_prenorm_h.float().cpu().numpy()[:M]
    assert np.isinf(h).sum() > 0, "the case must saturate the fp16 copy"
    print(f"  {int(np.isinf(h).sum())} elements of d_prenorm_h are infinite", flush=True)
    # dX with the pre-step W: non-finite in the same rows on both sides (fp16 operands)
    dx = db.input_grad(M).cpu().numpy()
    dx_ref = ob.input_grad(M)
    assert np.array_equal(~np.isfinite(dx).all(axis=1), ~np.isfinite(dx_ref).all(axis=1))
    ob.backward(x, O.Optimiser.adam(), O.Optimiser.adam(), M, 1e-3, 3.4e38, 1)
    db.backward(dev(x, True), abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3), 1)
    torch.cuda.synchronize()
    for n in ("dm_w", "dv_w", "master_w", "w"):
        a = db.get(n)
        assert np.all(np.isfinite(a)), f"{n}: {int((~np.isfinite(a)).sum())} non-finite elements"
    for n in ("dm_w", "dv_w", "master_w", "dm_b"):
        check(n, db.get(n), getattr(ob, n), FP16_TOL)
    assert np.array_equal(db.get("w"), db.get("master_w").astype(np.float16).astype(np.float32))
