"""DenseBlock hot-path benchmark on one MI355X (default: the headline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--settle-ms S] [--config c3|c2|c4|c5] [--no-cpu]
    python bench.py --copy-probe MIB      (counter calibration copy only)

Every step goes through the C ABI (libsoklyn_hip.so) with its inputs resident in HBM.

Single blocks (c3 = BASELINE config 3, the headline; c2 = config 2), one step =
  1. skl_dense_forward        Z = X.W + b, act           (GEMM, fused epilogue)
  2. skl_dense_error_from_sum dP = dY * act'(Z)           (element-wise + column sums)
  3. skl_dense_input_grad     dX = dP.W^T with the forward's W (the backward of a
                              single block, before its optimiser step)
  4. skl_dense_backward       dW = X^T.dP + optimiser on W, db + optimiser on b
  algorithmic work = 3 GEMMs x 2*M*K*N flops.
MLPs (c4 = config 4, c5 = config 5), one step = FeedForwardNetwork's train step
(src/ffn.rs:40-166): forward of every layer, output error, backward of the output
layer, then for each lower layer the hidden error from the updated layer above
followed by its own backward;
  algorithmic work = forward and dW of every layer + dX of layers 2..L.
Before the W warm-up steps the step runs untimed for at least --settle-ms of
wall time (default 250): under load the GPU's clocks take ~50 ms to reach their
steady state, and with few warm-up steps the timed steps would fall in that
ramp (C3: 855 TFLOP/s with 5 warm-up steps, 885-930 once settled).  The timed
region is still exactly K steps; the line reports the settle time and steps.
Inside the timed steps only the roofline GEMM kernel (the step's slowest GEMM,
named per configuration) carries HIP events, recorded by its own dispatch; every
GEMM kernel and every call is timed again in an untimed pass after them
(`kernel_ms`, `call_ms`).  Then, unless --power-ms 0, the step runs untimed while
amd-smi samples the socket power and graphics clock (`power`).
Prints one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"f16": 2516.6, "f32": 157.3}   # dense MFMA TFLOP/s: 256 CU x 2.4 GHz x {4096, 256} flop/clk/CU
HEADLINE = "DenseBlock fwd+bwd TFLOP/s & % MFMA peak (fp16, B=8192, 4096→4096)"

# activation / norm / loss / optimiser codes (reference ordinals, src/util/function.rs)
ACT_RELU, ACT_LEAKY, ACT_SIGMOID, ACT_SOFTMAX, ACT_SILU, ACT_MISH, ACT_IDENTITY = 2, 3, 1, 5, 6, 7, 0
NORM_RMS, NORM_LAYER = 1, 2
LOSS_CE, LOSS_BCE = 1, 2

CONFIGS = {
    # BASELINE.json configs[2] (headline) and configs[1]: single DenseBlocks
    "c3": dict(kind="block", M=8192, K=4096, N=4096, half=True, act=ACT_SILU, roof="dw_gemm",
               metric=HEADLINE,
               workload="DenseBlock fp16 mixed precision, X[8192x4096] f16, W[4096x4096] f16 copy of fp32 "
                        "He-normal master, SiLU, fwd+bwd(dX,dW)+Adam"),
    "c2": dict(kind="block", M=4096, K=1024, N=1024, half=False, act=ACT_RELU, roof="forward_gemm",
               metric="DenseBlock fwd+bwd TFLOP/s & % MFMA peak (fp32, B=4096, 1024→1024)",
               workload="DenseBlock fp32, X[4096x1024], W[1024x1024] He-normal, ReLU, fwd+bwd(dX,dW,db)+SGD"),
    # multi-layer train steps
    "c4": dict(kind="mlp", M=16384, dims=[3072, 2048, 2048, 2048, 2048, 10], x="uniform",
               hidden=dict(norm=NORM_RMS, act=ACT_MISH, mask_coeff=0.1), dropout=True,
               loss=LOSS_CE, loss_act=ACT_SOFTMAX, timed_layer=1,
               metric="MLP train step TFLOP/s & % MFMA peak (fp16, B=16384, 3072→2048⁴→10)",
               workload="5-layer MLP 3072->2048->2048->2048->2048->10 fp16 mixed precision, batch 16384, "
                        "RMSNorm + Mish + dropout 0.1 hidden, softmax CE, Adam; fwd+bwd+Adam train step"),
    "c5": dict(kind="mlp", M=12345, dims=[777, 1531, 3001, 13], x="normal2",
               hidden=dict(norm=NORM_LAYER, act=ACT_LEAKY, leaky=0.01), dropout=False,
               loss=LOSS_BCE, loss_act=ACT_SIGMOID, timed_layer=0,
               metric="MLP train step TFLOP/s & % MFMA peak (fp16, B=12345, 777→1531→3001→13)",
               workload="Ragged MLP 777->1531->3001->13 fp16 mixed precision, batch 12345, LayerNorm + "
                        "LeakyReLU(0.01) hidden, sigmoid BCE, Adam; fwd+bwd+Adam train step"),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    # ~50 ms of load before the timed steps: the GPU reaches its steady clocks only
    # after that (C3: 855 TFLOP/s with 5 warm-up steps, 885-895 with 50 or 200)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--settle-ms", type=float, default=250.0,
                   help="untimed steps before the warm-up until this much wall time has passed (clock ramp)")
    p.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-rows", type=int, default=0, help="rows of the CPU baseline sample (0 = auto)")
    p.add_argument("--power-ms", type=float, default=2000.0,
                   help="after the timed steps, run the step untimed this long while amd-smi samples the "
                        "socket power and graphics clock (0 = skip)")
    p.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                   help="only run a plain device-to-device copy of MIB MiB (counter calibration) and exit")
    return p.parse_args()


def copy_probe(mib: int) -> None:
    """A plain copy kernel of known size: HBM counters (FETCH_SIZE / WRITE_SIZE) read
    against it give the bytes-per-count factor used for roofline.traffic."""
    import torch
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "launches": 3}), flush=True)


def traffic_record(config: str, kernel: str):
    """HBM bytes per launch of the roofline kernel, from the committed rocprofv3 --pmc
    summary (FETCH_SIZE and WRITE_SIZE passes, each scaled by the copy-probe factor)."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(config, {}).get(kernel)
    except (OSError, ValueError):
        return None
    return rec


def mlp_flops(dims, M):
    """Forward and dW of every layer + dX of layers 2..L (the reference never forms dX
    of the network input)."""
    layer = [2.0 * M * dims[i] * dims[i + 1] for i in range(len(dims) - 1)]
    return 2 * sum(layer) + sum(layer[1:])


def mlp_inputs(cfg, g, rows):
    d0, d_last = cfg["dims"][0], cfg["dims"][-1]
    if cfg["x"] == "uniform":
        x = g.random((rows, d0), dtype=np.float32)
    else:                                   # N(0, 2): variance 2
        x = g.standard_normal((rows, d0)).astype(np.float32) * np.float32(np.sqrt(2.0))
    x = x.astype(np.float16).astype(np.float32)
    if cfg["loss"] == LOSS_CE:
        t = np.zeros((rows, d_last), np.float32)
        t[np.arange(rows), g.integers(0, d_last, rows)] = 1.0
    else:
        t = (g.random((rows, d_last)) > 0.5).astype(np.float32)
    return x, t


def mlp_weights(cfg, g):
    dims = cfg["dims"]
    return [(g.standard_normal((dims[i], dims[i + 1])) * np.sqrt(2.0 / dims[i])).astype(np.float32)
            for i in range(len(dims) - 1)]


def dropout_seeds(cfg, step):
    # weight ids of an fp16 training network built in order: 27 tensors per block (src/mlp.rs:45-421)
    from soklyn_amd import abi
    return [int(abi.load().skl_scramble_seed(step, 27 * i)) if cfg["dropout"] else 0
            for i in range(len(cfg["dims"]) - 1)]


def host_cpu():
    """The CPU the baseline runs on: its model (/proc/cpuinfo) and the cores this process may use."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "host_cores_available": len(os.sched_getaffinity(0))}


def _smi_sample(gpu: int = 0):
    """One `amd-smi metric -p -c` reading of GPU `gpu`: (socket power W, mean graphics clock MHz
    over the XCDs), or None when the tool or a field is unavailable."""
    import re
    import subprocess
    try:
        out = subprocess.run(["amd-smi", "metric", "-g", str(gpu), "-p", "-c"], capture_output=True,
                             text=True, timeout=5).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    p = re.search(r"SOCKET_POWER: (\d+(?:\.\d+)?) W", out)
    clks = [float(c) for c in re.findall(r"GFX_\d+:\s*\n\s*CLK: (\d+(?:\.\d+)?) MHz", out)]
    if not p or not clks:
        return None
    return float(p.group(1)), sum(clks) / len(clks)


def power_pass(step, ms: float, sync):
    """Run `step` untimed for `ms` of wall time while a thread samples amd-smi; returns the mean
    socket power and graphics clock over the samples after the first 0.5 s (the tool's power
    reading is a running average that lags the load), or None."""
    import threading
    samples, stop = [], threading.Event()
    t0 = time.perf_counter()

    def sampler():
        while not stop.is_set():
            r = _smi_sample()
            if r is None:
                return
            samples.append((time.perf_counter() - t0, *r))

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            step()
        sync()
    stop.set()
    th.join(timeout=10)
    kept = [s for s in samples if s[0] >= 0.5]
    if not kept:
        return None
    return {"socket_w": round(sum(s[1] for s in kept) / len(kept), 1),
            "gfx_mhz": round(sum(s[2] for s in kept) / len(kept), 1), "samples": len(kept),
            "source": "amd-smi metric -p -c during an untimed pass of the same step after the timed ones"}


def cpu_baseline_block(cfg, rows: int, reps: int = 3):
    """The oracle (C restatement, fp32, OpenMP over the host cores) on the same step:
    one warm-up pass, then the median of `reps` timed passes."""
    from oracle import oracle as O
    K, N = cfg["K"], cfg["N"]
    g = np.random.default_rng(0)
    w = (g.standard_normal((K, N)) * np.sqrt(2.0 / K)).astype(np.float32)
    x = g.standard_normal((rows, K)).astype(np.float32)
    s = (g.standard_normal((rows, N)) * 512).astype(np.float32)
    ob = O.OracleBlock(K, N, rows, w, act=cfg["act"])
    opt = O.Optimiser.adam() if cfg["half"] else O.Optimiser.sgd()

    def one(step):
        t0 = time.perf_counter()
        ob.forward(x, rows)
        ob.error_from_sum(s, rows)
        ob.input_grad(rows)
        ob.backward(x, opt, opt, rows, 1e-3, 3.4e38, step)
        return time.perf_counter() - t0

    one(1)
    times = sorted(one(2 + i) for i in range(reps))
    dt = times[len(times) // 2]
    flops = 3 * 2.0 * rows * K * N
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": O.num_threads(), "kind": "port",
            **host_cpu(),
            "sample": f"{rows} of {cfg['M']} batch rows of the same step (fwd, act', dW+update, dX) in fp32 "
                      f"on the oracle (OpenMP, {O.num_threads()} threads); median of {reps} passes after one "
                      f"warm-up, {dt:.2f} s per pass"}


def cpu_baseline_mlp(cfg, rows: int, reps: int = 3):
    """The oracle's FeedForwardNetwork train step (fp32) on `rows` of the batch."""
    from oracle import oracle as O
    g = np.random.default_rng(0)
    dims = cfg["dims"]
    ws = mlp_weights(cfg, g)
    x, t = mlp_inputs(cfg, g, rows)
    L = len(dims) - 1
    obs = [O.OracleBlock(dims[i], dims[i + 1], rows, ws[i], **(cfg["hidden"] if i < L - 1 else
                                                                dict(act=ACT_IDENTITY))) for i in range(L)]
    opt = O.Optimiser.adam()

    def one(step):
        seeds = dropout_seeds(cfg, step)
        t0 = time.perf_counter()
        cur, outs = x, []
        for ob, sd in zip(obs, seeds):
            cur = ob.forward(cur, rows, cfg["dropout"], sd)
            outs.append(cur)
        obs[L - 1].output_error(t, cfg["loss"], cfg["loss_act"])
        obs[L - 1].backward(outs[L - 2], opt, opt, rows, 1e-3, 3.4e38, step)
        for i in range(L - 2, -1, -1):
            obs[i].hidden_error(obs[i + 1], rows)
            obs[i].backward(outs[i - 1] if i > 0 else x, opt, opt, rows, 1e-3, 3.4e38, step)
        return time.perf_counter() - t0

    one(1)
    times = sorted(one(2 + i) for i in range(reps))
    dt = times[len(times) // 2]
    return {"value": round(mlp_flops(dims, rows) / dt / 1e12, 6), "unit": "TFLOP/s", "cores": O.num_threads(),
            "kind": "port", **host_cpu(),
            "sample": f"{rows} of {cfg['M']} batch rows of the same train step (all layers fwd, loss, bwd + Adam) "
                      f"in fp32 on the oracle (OpenMP, {O.num_threads()} threads); median of {reps} passes after "
                      f"one warm-up, {dt:.2f} s per pass"}


def timing_events(n):
    """n (start, stop) pairs of timing events, each recorded once so its HIP event exists."""
    import torch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for a, b in evs:
        a.record()
        b.record()
    return evs


class BlockBench:
    """Single DenseBlock: forward -> error_from_sum -> input_grad -> backward."""
    calls = ("forward", "error_from_sum", "input_grad", "backward")
    # GEMM kernels timed alone (the roofline candidates): forward (+bias, act), dW (+ the
    # optimiser step on W in its epilogue) and dX
    gemms = ("forward_gemm", "dw_gemm", "dx_gemm")

    def __init__(self, cfg, ctx, stream):
        import torch
        from soklyn_amd import abi
        from soklyn_amd.devblock import DeviceBlock
        M, K, N, half = cfg["M"], cfg["K"], cfg["N"], cfg["half"]
        dt = torch.float16 if half else torch.float32
        g = np.random.default_rng(1)
        w = (g.standard_normal((K, N)) * np.sqrt(2.0 / K)).astype(np.float32)
        self.blk = DeviceBlock(ctx, K, N, M, w, half=half, act=cfg["act"], master_w=w if half else None,
                               b=(g.standard_normal((1, N)) * 0.01).astype(np.float32))
        self.x = torch.randn((M, K), device="cuda", dtype=torch.float32).to(dt)
        self.dy = torch.randn((M, N), device="cuda", dtype=torch.float32) * 512.0
        self.dx = torch.empty((M, K), device="cuda", dtype=torch.float32)
        opt = abi.adam(0.9, 0.999, 1e-8) if half else abi.sgd(0.0)
        self.tc = abi.train_ctx(opt, opt, M, 1e-3 if half else 1e-2)
        self.M = M
        self.step_no = 0
        self.flops = 3 * 2.0 * M * K * N
        self.kernel_flops = {g: 2.0 * M * K * N for g in self.gemms}
        self.roof = cfg["roof"]   # the slowest GEMM of the step (checked against the untimed pass)
        self.stream, self.ctx = stream, ctx
        # error_from_sum is one element-wise kernel: its algorithmic HBM bytes (the
        # activation derivative reads predrop for sigmoid / ReLU / leaky ReLU / tanh /
        # SiLU and preact for SiLU / Mish; the mask always)
        act, ts = cfg["act"], 2 if half else 4
        reads = 4 + ts * (int(act in (ACT_SIGMOID, ACT_RELU, ACT_LEAKY, 4, ACT_SILU))
                          + int(act in (ACT_SILU, ACT_MISH)) + 1)
        writes = 4 + 4 + (2 if half else 0)       # grad, d_prenorm (fp32), d_prenorm_h (fp16 blocks)
        self.hbm_bytes = {"error_from_sum": float(M) * N * (reads + writes)}

    def step(self, ev=None, gev=None):
        # ev: per-call (start, end) HIP events on the launch stream (a diagnostic pass
        # after the timed steps); gev: {GEMM name: (start, end)} events the library records
        # around that GEMM kernel alone, carried by its dispatch
        self.step_no += 1
        b, M = self.blk, self.M
        fns = (lambda: b.forward(self.x, M), lambda: b.error_from_sum(self.dy, M),
               lambda: b.input_grad(M, self.dx), lambda: b.backward(self.x, self.tc, self.step_no))
        gemm_of = {0: "forward_gemm", 2: "dx_gemm", 3: "dw_gemm"}   # call index -> GEMM name
        for i, fn in enumerate(fns):
            if gev is not None and gemm_of.get(i) in gev:
                self.ctx.time_next_gemm(*gev[gemm_of[i]])
            if ev is not None:
                ev[i][0].record(self.stream)
            fn()
            if ev is not None:
                ev[i][1].record(self.stream)


class MlpBench:
    """FeedForwardNetwork train step over DeviceBlocks (src/ffn.rs:40-166 order)."""

    def __init__(self, cfg, ctx, stream):
        import torch
        from soklyn_amd import abi
        from soklyn_amd.devblock import DeviceBlock
        self.cfg, self.abi, self.stream = cfg, abi, stream
        dims, M = cfg["dims"], cfg["M"]
        g = np.random.default_rng(1)
        ws = mlp_weights(cfg, g)
        L = len(dims) - 1
        self.blocks = [DeviceBlock(ctx, dims[i], dims[i + 1], M, ws[i], half=True, master_w=ws[i],
                                   **(cfg["hidden"] if i < L - 1 else dict(act=ACT_IDENTITY)))
                       for i in range(L)]
        x, t = mlp_inputs(cfg, g, M)
        self.x = torch.from_numpy(x).cuda().half()
        self.t = torch.from_numpy(t).cuda().half()
        self.tc = abi.train_ctx(abi.adam(), abi.adam(), M, 1e-3)
        self.M, self.L = M, L
        self.step_no = 0
        self.flops = mlp_flops(dims, M)
        # the roofline kernel: the GEMM of the hidden error of layer `timed_layer`, dX
        # through the weights of the layer above it (the call also runs the error
        # kernel, then the layer's dW and optimiser step)
        k = cfg["timed_layer"]
        self.timed = f"hidden_error_gemm_layer{k}"
        self.calls = (f"backward_hidden_layer{k}",)
        self.gemms = (self.timed,)
        self.roof = self.timed
        self.kernel_flops = {self.timed: 2.0 * M * dims[k + 1] * dims[k + 2]}
        self.hbm_bytes = {}
        self.ctx = ctx

    def step(self, ev=None, gev=None):
        self.step_no += 1
        cfg, b, M, L = self.cfg, self.blocks, self.M, self.L
        seeds = dropout_seeds(cfg, self.step_no)
        cur = self.x
        for blk, sd in zip(b, seeds):
            cur = blk.forward(cur, M, cfg["dropout"], sd)
        b[L - 1].output_error(self.t, cfg["loss"], cfg["loss_act"])
        b[L - 1].backward(b[L - 2].out, self.tc, self.step_no)
        for i in range(L - 2, -1, -1):
            timed = i == cfg["timed_layer"]
            if timed and gev is not None:
                self.ctx.time_next_gemm(*gev[self.timed])
            if timed and ev is not None:
                ev[0][0].record(self.stream)
            # gpu_hidden_layer_backward_pass (ffn.rs:156 -> mlp.rs:728): hidden error, then dW
            b[i].backward_hidden(b[i + 1], b[i - 1].out if i > 0 else self.x, self.tc, self.step_no)
            if timed and ev is not None:
                ev[0][1].record(self.stream)


def main():
    args = parse()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)
    import torch
    from soklyn_amd import abi

    cfg = CONFIGS[args.config]
    torch.manual_seed(0)
    stream = torch.cuda.Stream()          # explicit, default priority (stream 0 has handle 0)
    torch.cuda.set_stream(stream)
    ctx = abi.Context(0, 16)
    ctx.set_stream(stream.cuda_stream)
    ctx.set_sync(False)
    bench = BlockBench(cfg, ctx, stream) if cfg["kind"] == "block" else MlpBench(cfg, ctx, stream)
    calls, gemms = bench.calls, bench.gemms

    # events first, so nothing but the warm-up steps runs between warm-up and timing.
    # In the timed steps only the roofline GEMM kernel carries events: each kernel-carried
    # pair leaves the GPU idle for ~5 us around its kernel (three pairs cost a C3 step
    # 1.8%); every GEMM is timed in the untimed pass after them.
    evs = [timing_events(len(calls)) for _ in range(args.steps)]
    gevs = [dict(zip(gemms, timing_events(len(gemms)))) for _ in range(args.steps)]
    rev = [{bench.roof: timing_events(1)[0]} for _ in range(args.steps)]
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    settle_steps, t_settle = 0, time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms:
        for _ in range(4):
            bench.step()
        settle_steps += 4
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        bench.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for k in range(args.steps):
        bench.step(None, rev[k])      # only the roofline GEMM kernel carries events
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps
    value = bench.flops / (ms * 1e-3) / 1e12
    # Per-call and per-GEMM times come from a second, untimed pass: recorded inside the
    # timed steps, the 8 extra events of a C3 step cost ~3.5% of its time.
    for k in range(args.steps):
        bench.step(evs[k], gevs[k])
    torch.cuda.synchronize()

    def avg(table, names):
        return {c: sum(table[k][i][0].elapsed_time(table[k][i][1]) for k in range(args.steps)) / args.steps
                for i, c in enumerate(names)}
    call_ms = avg(evs, calls)     # each hot-path call in the step
    kern = {g: sum(gevs[k][g][0].elapsed_time(gevs[k][g][1]) for k in range(args.steps)) / args.steps
            for g in gemms}       # the GEMM kernels alone (untimed pass)
    roof_ms = sum(rev[k][bench.roof][0].elapsed_time(rev[k][bench.roof][1])
                  for k in range(args.steps)) / args.steps   # the roofline kernel in the timed steps
    # Socket power and graphics clock under this step (the GEMMs run at the board's power
    # limit, where the clock settles well below the 2.4 GHz of the published peak)
    power = power_pass(bench.step, args.power_ms, torch.cuda.synchronize) if args.power_ms > 0 else None

    # The roofline kernel: the step's slowest GEMM, timed inside the timed steps
    dom = bench.roof
    slowest = max(gemms, key=lambda k: kern[k])
    achieved = bench.kernel_flops[dom] / (roof_ms * 1e-3) / 1e12
    half = cfg.get("half", True)
    peak = PEAK["f16" if half else "f32"]
    trec = traffic_record(args.config, dom)
    config = {"workload": cfg["workload"], "M": cfg["M"]}
    if cfg["kind"] == "block":
        config.update(K=cfg["K"], N=cfg["N"])
    else:
        config.update(dims=cfg["dims"])
    config.update(gflop_per_step=round(bench.flops / 1e9, 3), pct_of_peak_step=round(100 * value / peak, 2),
                  wall_s=round(wall, 3))

    out = {
        "metric": cfg["metric"],
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"ms": args.settle_ms, "steps": settle_steps},
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if half else "f32",
        "data": "synthetic (seeded inputs and targets of the config's distributions, He-normal weights"
                + (", N(0,1)*512 upstream gradient)" if cfg["kind"] == "block" else ")"),
        "config": config,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4),
                     "traffic": trec["bytes_per_launch"] if trec else None,
                     "traffic_source": trec["source"] if trec else None, "kernel": dom,
                     "kernel_ms_timed": round(roof_ms, 4), "slowest_gemm_untimed_pass": slowest,
                     "kernel_ms": {k: round(v, 4) for k, v in kern.items()},
                     "call_ms": {k: round(v, 4) for k, v in call_ms.items()}},
    }
    if power is not None:
        # the dense fp16 / fp32 MFMA peak at the measured clock, for reading the roofline
        # fraction against the clock the power limit leaves
        power["peak_at_clock"] = round(peak * power["gfx_mhz"] / 2400.0, 1)
        power["kernel_frac_at_clock"] = round(achieved / power["peak_at_clock"], 4)
    out["power"] = power
    # bandwidth-bound calls made of one element-wise kernel: algorithmic bytes / call time
    if bench.hbm_bytes:
        out["hbm_kernels"] = {
            c: {"bytes": int(b), "ms": round(call_ms[c], 4), "GB/s": round(b / (call_ms[c] * 1e-3) / 1e9, 1),
                "frac_of_8TB/s": round(b / (call_ms[c] * 1e-3) / 8e12, 4)}
            for c, b in bench.hbm_bytes.items()}
    if not args.no_cpu:
        if cfg["kind"] == "block":
            out["cpu_baseline"] = cpu_baseline_block(cfg, args.cpu_rows or cfg["M"])
        else:
            # a quarter of the batch: 10-20 s of the oracle on the host cores
            out["cpu_baseline"] = cpu_baseline_mlp(cfg, args.cpu_rows or cfg["M"] // 4)
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
