"""The C++ host API end to end on the GPU: FeedForwardNetwork training steps driven by
soklyn_tool (DenseBlock::new_with_config with InitHeNormalFunc, forward with dropout
seeded by scramble_seed(step, weight id), compute_loss, backward_output and
backward_hidden in the order of src/ffn.rs:113-166), checked against the oracle run on
the same initial weights, inputs and seeds; the tensor-id sequence of
src/mlp.rs:46-421 (23 ids per fp32 training block, 27 per fp16 one); and the trained
network's checkpoint (src/io/save.rs): the tool saves it, reloads it into blocks and
checks every tensor and the forward bit for bit, and the file itself is checked here
with the `safetensors` library and against the reference's header layout.
"""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from soklyn_amd import abi
from tests.helpers import FP16_TOL, FP32_TOL, check, check_adam_update, f16, rng
from tests.test_gpu_ffn import oracle_step
from tests.test_safetensors_cpu import serde_pretty_header

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.path.join(ROOT, "soklyn_amd", "host", "soklyn_tool")


def tool(*args) -> str:
    print("soklyn_tool", *args, flush=True)
    p = subprocess.run([TOOL, *map(str, args)], capture_output=True, text=True, timeout=110)
    assert p.returncode == 0, p.stdout + p.stderr
    return p.stdout


def test_tensor_ids_per_block():
    got = dict(l.split() for l in tool("ids").strip().splitlines())
    # training: linear 2 + 4 moments, norm 2 + 4, caches 6, grads 4, mask 1 (+ 2 + 2 masters for fp16)
    assert got == {"f32_train": "23", "f16_train": "27", "f32_infer": "11", "f16_infer": "15"}


def run_scenario(tmp, *, dtype, dims, batch, steps, norm, act, leaky, mask_coeff, loss, loss_act, opt, lr,
                 dropout, init_seed, x, t):
    spec = dict(dtype=dtype, dims=",".join(map(str, dims)), batch=batch, steps=steps, norm=norm, act=act,
                leaky=leaky, mask_coeff=mask_coeff, loss=loss, loss_act=loss_act, lr=lr, dropout=int(dropout),
                init_seed=init_seed, **opt)
    with open(os.path.join(tmp, "spec.txt"), "w") as fh:
        fh.write("".join(f"{k}={v}\n" for k, v in spec.items()))
    x.astype(np.float32).tofile(os.path.join(tmp, "x.bin"))
    t.astype(np.float32).tofile(os.path.join(tmp, "t.bin"))
    out = tool("train", tmp)
    assert "checkpoint round trip OK" in out
    L = len(dims) - 1
    ids = [int(l) for l in open(os.path.join(tmp, "ids.txt")).read().split()]
    w0 = [np.fromfile(os.path.join(tmp, f"w{i}_init.bin"), np.float32).reshape(dims[i], dims[i + 1])
          for i in range(L)]
    res = {}
    for i in range(L):
        for n in ("out", "w", "master_w", "b", "dv_w", "dm_w", "dv_b", "grad", "d_prenorm", "mask"):
            path = os.path.join(tmp, f"{n}{i}.bin")
            if os.path.exists(path):
                res[(n, i)] = np.fromfile(path, np.float32)
    check_checkpoint(os.path.join(tmp, "net.safetensors"), dims, dtype, res, steps)
    return ids, w0, res


def check_checkpoint(path, dims, dtype, res, steps):
    """save.rs:227-345: names, shapes, dtypes, data order and values of the written file."""
    from safetensors import safe_open
    from safetensors.numpy import load_file
    t = load_file(path)
    tdt = "F16" if dtype == "f16" else "F32"
    expect, off = {}, 0
    for i in range(len(dims) - 1):
        K, N, pre = dims[i], dims[i + 1], f"layer{i + 1}."
        entries = [("w", tdt, (K, N)), ("b", tdt, (N,)), ("norm_w", tdt, (N,)), ("norm_b", tdt, (N,)),
                   ("dv_w", "F32", (K, N)), ("dv_b", "F32", (N,)), ("dm_w", "F32", (K, N)), ("dm_b", "F32", (N,)),
                   ("dv_norm_w", "F32", (N,)), ("dv_norm_b", "F32", (N,)), ("dm_norm_w", "F32", (N,)),
                   ("dm_norm_b", "F32", (N,))]
        if dtype == "f16":
            entries += [("master_w", "F32", (K, N)), ("master_b", "F32", (1, N)), ("master_norm_w", "F32", (1, N)),
                        ("master_norm_b", "F32", (1, N))]
        for n, dt, shape in entries:
            nbytes = int(np.prod(shape)) * (2 if dt == "F16" else 4)
            expect[pre + n] = (dt, shape, off, off + nbytes)
            off += nbytes
            assert t[pre + n].shape == shape and t[pre + n].dtype == (np.float16 if dt == "F16" else np.float32), n
        for n in ("w", "b", "dv_w", "dm_w", "dv_b") + (("master_w",) if dtype == "f16" else ()):
            assert np.array_equal(t[pre + n].astype(np.float32).reshape(-1), res[(n, i)]), f"layer {i} {n}"
    assert set(t) == set(expect)
    blob = open(path, "rb").read()
    n = int(np.frombuffer(blob[:8], "<u8")[0])
    assert blob[8:8 + n] == serde_pretty_header(expect, {"steps": str(steps)})
    assert len(blob) == 8 + n + off
    with safe_open(path, "np") as f:
        assert f.metadata() == {"steps": str(steps)}


def oracle_net(dims, batch, half, w0, hidden_kw):
    obs = []
    for i in range(len(dims) - 1):
        kw = dict(hidden_kw) if i < len(dims) - 2 else dict(act=abi.ACT_IDENTITY)
        obs.append(O.OracleBlock(dims[i], dims[i + 1], batch, w0[i], half=half, master_w=w0[i] if half else None,
                                 **kw))
    return obs


def compare(obs, res, tol, half, masks):
    for i, ob in enumerate(obs):
        for n in ("out", "grad", "d_prenorm", "dv_w", "dm_w", "dv_b", "master_w" if half else "w"):
            ref = np.asarray(getattr(ob, n), np.float32).reshape(-1)
            check(f"layer {i} {n}", res[(n, i)], ref, tol)
        if masks and i < len(obs) - 1:
            assert np.array_equal(res[("mask", i)], np.asarray(ob.mask, np.float32).reshape(-1)), f"layer {i} mask"


def test_ffn_fp32_sgd_two_steps(tmp_path):
    """784 -> 128 (ReLU) -> 10 (softmax CE), fp32, SGD with momentum, two steps (config 1's shape)."""
    dims, M, steps = [784, 128, 10], 64, 2
    g = rng(201)
    x = g.random((M, 784), dtype=np.float32)
    t = np.zeros((M, 10), np.float32)
    t[np.arange(M), g.integers(0, 10, M)] = 1
    ids, w0, res = run_scenario(str(tmp_path), dtype="f32", dims=dims, batch=M, steps=steps, norm=0,
                                act=abi.ACT_RELU, leaky=0.0, mask_coeff=0.0, loss=abi.LOSS_CE,
                                loss_act=abi.ACT_SOFTMAX, opt=dict(opt="sgd", v=0.9, nesterov=0), lr=0.01,
                                dropout=False, init_seed=42, x=x, t=t)
    # He-normal: sigma = sqrt(2 / fan_in)
    assert abs(w0[0].std() / np.sqrt(2 / 784) - 1) < 0.05
    obs = oracle_net(dims, M, False, w0, dict(act=abi.ACT_RELU))
    for step in range(1, steps + 1):
        seeds = [O.scramble_seed(step, i) for i in ids]
        oracle_step(obs, x, t, M, abi.LOSS_CE, abi.ACT_SOFTMAX, O.Optimiser.sgd(0.9), 0.01, step, False, seeds)
    compare(obs, res, FP32_TOL, False, masks=False)


def test_ffn_fp16_rms_mish_dropout_adam_two_steps(tmp_path):
    """96 -> 64 -> 64 -> 10, RMSNorm + Mish + dropout 0.1 hidden layers, CE, Adam, fp16 (config 4's
    layer recipe at a small size); the dropout masks must match bit for bit."""
    dims, M, steps = [96, 64, 64, 10], 256, 2
    g = rng(202)
    x = f16(g.random((M, 96), dtype=np.float32))
    t = np.zeros((M, 10), np.float32)
    t[np.arange(M), g.integers(0, 10, M)] = 1
    ids, w0, res = run_scenario(str(tmp_path), dtype="f16", dims=dims, batch=M, steps=steps, norm=abi.NORM_RMS,
                                act=abi.ACT_MISH, leaky=0.0, mask_coeff=0.1, loss=abi.LOSS_CE,
                                loss_act=abi.ACT_SOFTMAX, opt=dict(opt="adam", m=0.9, v=0.999, eps=1e-8),
                                lr=1e-3, dropout=True, init_seed=7, x=x, t=t)
    assert ids[1] - ids[0] == 27 and ids[2] - ids[1] == 27   # one fp16 training block apart
    obs = oracle_net(dims, M, True, w0, dict(norm=abi.NORM_RMS, act=abi.ACT_MISH, mask_coeff=0.1))
    for step in range(1, steps + 1):
        seeds = [O.scramble_seed(step, i) for i in ids]
        oracle_step(obs, x, t, M, abi.LOSS_CE, abi.ACT_SOFTMAX, O.Optimiser.adam(), 1e-3, step, True, seeds)
    compare(obs, res, FP16_TOL, True, masks=True)


def test_convert_f16_train_convert_f32_round_trip(tmp_path):
    """DenseBlock<f32>::convert_f16 (mlp.rs:835-856, ParamState::cast_f16 at mlp.rs:204-219), one fp16
    Adam step, DenseBlock<f16>::convert_f32 (mlp.rs:868-888, cast_f32 at mlp.rs:186-202), one fp32
    forward: the casts bit for bit, the step and the final forward against the oracle."""
    K, N, M = 96, 80, 64
    d = str(tmp_path)
    g = rng(301)
    x = g.standard_normal((M, K)).astype(np.float32)
    t = g.standard_normal((M, N)).astype(np.float32)
    x.tofile(os.path.join(d, "x.bin"))
    t.tofile(os.path.join(d, "t.bin"))
    assert "convert round trip done" in tool("convert", d, K, N, M, 1234)

    def ld(n, shape=None):
        a = np.fromfile(os.path.join(d, n + ".bin"), np.float32)
        return a.reshape(shape) if shape else a

    w32 = ld("w32_init", (K, N))
    assert w32.std() > 0 and np.all(ld("mask32_init") == 1.0)
    # convert_f16: master = the fp32 original, w = f16(RNE) of it, norm_w = 1 in both, mask cast
    assert np.array_equal(ld("master_w16", (K, N)), w32)
    assert np.array_equal(ld("w16", (K, N)), f16(w32))
    assert np.all(ld("norm_w16") == 1.0) and np.all(ld("master_norm_w16") == 1.0)
    assert np.all(ld("mask16") == 1.0)

    # the fp16 step against the oracle on the same weights (convert_f16 route: master = w32)
    ob = O.OracleBlock(K, N, M, w32, half=True, master_w=w32, norm=abi.NORM_RMS, act=abi.ACT_SILU)
    xh, th = f16(x), f16(t)
    ob.forward(xh, M)
    ob.output_error(th, abi.LOSS_MSE, abi.ACT_IDENTITY)
    ob.backward(xh, O.Optimiser.adam(), O.Optimiser.adam(), M, 1e-3, 3.4e38, 1)
    check("out (fp16 step)", ld("out16", (M, N)), ob.out, FP16_TOL)
    check("d_prenorm (fp16 step)", ld("d_prenorm16", (M, N)), ob.d_prenorm, FP16_TOL)
    check("dm_w (fp16 step)", ld("dm_w16_step", (K, N)), ob.dm_w, FP16_TOL)
    check("dv_w (fp16 step)", ld("dv_w16_step", (K, N)), ob.dv_w, FP16_TOL)
    m_step = ld("master_w16_step", (K, N))
    check_adam_update("master_w update", w32, m_step, ld("dm_w16_step", (K, N)), ld("dv_w16_step", (K, N)), 1e-3, 1,
                      ob.master_w - w32, ob.dm_w)
    assert np.array_equal(ld("w16_step", (K, N)), f16(m_step))

    # convert_f32: w = the fp32 master, moments carried over, caches cast f16 -> f32 exactly
    w_back = ld("w32_back", (K, N))
    assert np.array_equal(w_back, m_step)
    assert np.array_equal(ld("norm_w32_back"), ld("master_norm_w16_step"))
    assert np.array_equal(ld("b32_back"), ld("master_b16_step"))
    assert np.array_equal(ld("norm_b32_back"), ld("master_norm_b16_step"))
    assert np.array_equal(ld("dm_w32_back", (K, N)), ld("dm_w16_step", (K, N)))
    assert np.array_equal(ld("dv_w32_back", (K, N)), ld("dv_w16_step", (K, N)))
    assert np.array_equal(ld("out32_back", (M, N)), ld("out16", (M, N)))

    # and the converted block computes in fp32
    o32 = O.OracleBlock(K, N, M, w_back, norm=abi.NORM_RMS, act=abi.ACT_SILU, b=ld("b32_back"))
    o32.norm_w[:] = ld("norm_w32_back").reshape(1, N)
    o32.norm_b[:] = ld("norm_b32_back").reshape(1, N)
    o32.forward(xh, M)
    check("out (fp32 forward after convert_f32)", ld("out32_fwd", (M, N)), o32.out, FP32_TOL)
