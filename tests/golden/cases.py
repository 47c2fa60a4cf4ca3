"""Tiny seeded DenseBlock cases whose oracle outputs are committed as golden vectors
(tests/golden/oracle_tiny.npz, written by tests/golden/make_oracle_vectors.py).

Each case is one training step through the C-ABI entry points in the reference's
order: forward (all layers) -> output error (or an upstream gradient) -> backward of
the last layer -> hidden error + backward of the layer below -> dX of the input.
`run(case, make_block)` drives either the oracle or the device through the same
sequence and returns the named results; the inputs come from the case's seed.
"""
from __future__ import annotations

import zlib

import numpy as np

# ordinals as in include/soklyn_hip.h
NORM_NONE, NORM_RMS, NORM_LAYER, NORM_BATCH = 0, 1, 2, 3
ACT_ID, ACT_SIGMOID, ACT_RELU, ACT_LEAKY, ACT_TANH, ACT_SOFTMAX, ACT_SILU, ACT_MISH = range(8)
LOSS_MSE, LOSS_CE, LOSS_BCE = 0, 1, 2

CASES = {
    # single block, ragged, upstream gradient, SGD + Nesterov momentum
    "f32_relu_sgd": dict(half=False, dims=[7, 5], M=6, layers=[dict(act=ACT_RELU)], upstream=True,
                         opt=("sgd", 0.9, True), lr=0.05, dropout=False),
    # fp16 block: RMSNorm + Mish + dropout, Adam
    "f16_rms_mish_dropout_adam": dict(half=True, dims=[16, 24], M=8,
                                      layers=[dict(norm=NORM_RMS, act=ACT_MISH, mask_coeff=0.25)], upstream=True,
                                      opt=("adam",), lr=1e-2, dropout=True),
    # two fp32 layers: LayerNorm + LeakyReLU hidden, BCE / sigmoid head, Adam
    "f32_ln_leaky_bce_2layer": dict(half=False, dims=[9, 12, 3], M=5,
                                    layers=[dict(norm=NORM_LAYER, act=ACT_LEAKY, leaky=0.01), dict(act=ACT_ID)],
                                    upstream=False, loss=(LOSS_BCE, ACT_SIGMOID), opt=("adam",), lr=1e-2,
                                    dropout=False),
    # two fp16 layers: BatchNorm + Tanh hidden, CE / softmax head, SGD
    "f16_bn_tanh_ce_2layer": dict(half=True, dims=[10, 6, 4], M=7,
                                  layers=[dict(norm=NORM_BATCH, act=ACT_TANH), dict(act=ACT_ID)], upstream=False,
                                  loss=(LOSS_CE, ACT_SOFTMAX), opt=("sgd", 0.0, False), lr=0.1, dropout=False),
}

RESULTS = ("out", "predrop", "preact", "mask", "grad", "d_prenorm", "dv_w", "dm_w", "dv_b", "dm_b")


def f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def inputs(name: str) -> dict:
    """Seeded inputs of a case: weights, biases, x, upstream gradient or target, seeds."""
    c = CASES[name]
    g = np.random.default_rng(zlib.crc32(name.encode()))
    dims, M, half = c["dims"], c["M"], c["half"]
    d = {}
    for i in range(len(dims) - 1):
        w = (g.standard_normal((dims[i], dims[i + 1])) * np.sqrt(2.0 / dims[i])).astype(np.float32)
        b = (g.standard_normal((1, dims[i + 1])) * 0.1).astype(np.float32)
        d[f"w{i}"], d[f"b{i}"] = w, (f16(b) if half else b)
    x = g.standard_normal((M, dims[0])).astype(np.float32)
    d["x"] = f16(x) if half else x
    if c["upstream"]:
        d["s"] = (g.standard_normal((M, dims[-1])) * 512).astype(np.float32)
    else:
        loss = c["loss"][0]
        t = np.zeros((M, dims[-1]), np.float32)
        if loss == LOSS_CE:
            t[np.arange(M), g.integers(0, dims[-1], M)] = 1
        else:
            t = (g.random((M, dims[-1])) > 0.5).astype(np.float32)
        d["t"] = t
    d["seeds"] = np.array([1234567 + 89 * i for i in range(len(dims) - 1)], np.uint32)
    return d


def run(name: str, d: dict, make_block, opt_fn, train_fn, to_dev, from_dev) -> dict:
    """One step of case `name` on inputs `d`.  make_block(K, N, M, w, half, b, **layer_kw)
    builds an oracle or device block; opt_fn(spec) an optimiser; train_fn(opt, M, lr) the
    training context argument; to_dev / from_dev move arrays.  Returns {name: array}."""
    c = CASES[name]
    dims, M, half = c["dims"], c["M"], c["half"]
    L = len(dims) - 1
    blocks = [make_block(dims[i], dims[i + 1], M, d[f"w{i}"], half, d[f"b{i}"], **c["layers"][i]) for i in range(L)]
    opt = opt_fn(c["opt"])
    train = train_fn(opt, M, c["lr"])
    x = to_dev(d["x"], half)
    cur, outs = x, []
    for i, blk in enumerate(blocks):
        cur = blk.forward(cur, M, c["dropout"], int(d["seeds"][i]))
        outs.append(cur)
    last = blocks[-1]
    if c["upstream"]:
        last.error_from_sum(to_dev(d["s"], False), M)
    else:
        last.output_error(to_dev(d["t"], half), c["loss"][0], c["loss"][1])
    res = {}
    head_in = outs[L - 2] if L > 1 else x
    last.backward(head_in, *train)
    for i in range(L - 2, -1, -1):
        blocks[i].hidden_error(blocks[i + 1], M)
        blocks[i].backward(outs[i - 1] if i > 0 else x, *train)
    res["dx"] = from_dev(blocks[0].input_grad(M))
    for i, blk in enumerate(blocks):
        for n in RESULTS + (("master_w",) if half else ("w",)):
            res[f"{n}{i}"] = np.asarray(blk.get(n) if hasattr(blk, "get") else getattr(blk, n), np.float32).copy()
    return res
