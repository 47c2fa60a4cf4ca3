"""Headline benchmark: fp16 DenseBlock fwd+bwd+Adam at B=8192, 4096->4096 on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c3|c2] [--no-cpu]
    python bench.py --copy-probe MIB      (counter calibration copy only)

One step = one pass of the DenseBlock hot path over one batch, all through the
C ABI (libsoklyn_hip.so), inputs resident in HBM:
  1. skl_dense_forward        Z = X.W + b, SiLU          (GEMM, fused epilogue)
  2. skl_dense_error_from_sum dP = dY * SiLU'(Z)          (element-wise)
  3. skl_dense_backward       dW = X^T.dP + Adam on W, db + Adam on b
  4. skl_dense_input_grad     dX = dP.W^T (updated W, src/ffn.rs:142-163 order)
Algorithmic work = 3 GEMMs x 2*M*K*N flops.  Prints one JSON line.
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
CONFIGS = {
    # BASELINE.json configs[2] (headline) and configs[1]
    "c3": dict(M=8192, K=4096, N=4096, half=True, act=6, workload="DenseBlock fp16 mixed precision, "
               "X[8192x4096] f16, W[4096x4096] f16 copy of fp32 He-normal master, SiLU, fwd+bwd(dX,dW)+Adam"),
    "c2": dict(M=4096, K=1024, N=1024, half=False, act=2, workload="DenseBlock fp32, X[4096x1024], "
               "W[1024x1024] He-normal, ReLU, fwd+bwd(dX,dW,db)+SGD"),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="c3", choices=sorted(CONFIGS))
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-rows", type=int, default=0, help="rows of the CPU baseline sample (0 = auto)")
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


def cpu_baseline(cfg, rows: int, reps: int = 3):
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
        ob.backward(x, opt, opt, rows, 1e-3, 3.4e38, step)
        ob.input_grad(rows)
        return time.perf_counter() - t0

    one(1)
    times = sorted(one(2 + i) for i in range(reps))
    dt = times[len(times) // 2]
    flops = 3 * 2.0 * rows * K * N
    return {"value": round(flops / dt / 1e12, 6), "unit": "TFLOP/s", "cores": O.num_threads(), "kind": "port",
            "sample": f"{rows} of {cfg['M']} batch rows of the same step (fwd, act', dW+update, dX) in fp32 "
                      f"on the oracle; median of {reps} passes after one warm-up, {dt:.2f} s per pass"}


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
    from soklyn_amd.devblock import DeviceBlock

    cfg = CONFIGS[args.config]
    M, K, N, half = cfg["M"], cfg["K"], cfg["N"], cfg["half"]
    dt = torch.float16 if half else torch.float32
    torch.manual_seed(0)
    stream = torch.cuda.Stream()          # explicit, default priority (stream 0 has handle 0)
    torch.cuda.set_stream(stream)
    ctx = abi.Context(0, 16)
    ctx.set_stream(stream.cuda_stream)
    ctx.set_sync(False)

    g = np.random.default_rng(1)
    w = (g.standard_normal((K, N)) * np.sqrt(2.0 / K)).astype(np.float32)
    blk = DeviceBlock(ctx, K, N, M, w, half=half, act=cfg["act"], master_w=w if half else None,
                      b=(g.standard_normal((1, N)) * 0.01).astype(np.float32))
    x = torch.randn((M, K), device="cuda", dtype=torch.float32).to(dt)
    dy = torch.randn((M, N), device="cuda", dtype=torch.float32) * 512.0
    dx = torch.empty((M, K), device="cuda", dtype=torch.float32)
    opt = abi.adam(0.9, 0.999, 1e-8) if half else abi.sgd(0.0)
    tc = abi.train_ctx(opt, opt, M, 1e-3 if half else 1e-2)
    step_no = [0]

    calls = ("forward_gemm", "error_elementwise", "dw_gemm_adam", "dx_gemm")

    def step(ev=None):
        # ev: per-call (start, end) HIP events on the launch stream, recorded
        # inside the timed steps so each call is timed in the step's own context
        step_no[0] += 1
        fns = (lambda: blk.forward(x, M), lambda: blk.error_from_sum(dy, M),
               lambda: blk.backward(x, tc, step_no[0]), lambda: blk.input_grad(M, dx))
        for i, fn in enumerate(fns):
            if ev is not None:
                ev[i][0].record(stream)
            fn()
            if ev is not None:
                ev[i][1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in calls]
           for _ in range(args.steps)]
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for k in range(args.steps):
        step(evs[k])
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps
    flops = 3 * 2.0 * M * K * N
    value = flops / (ms * 1e-3) / 1e12
    # average duration of each call over the timed steps (forward and dX are one
    # kernel launch each at these shapes; dW+Adam adds the bias column sums)
    kern = {c: sum(evs[k][i][0].elapsed_time(evs[k][i][1]) for k in range(args.steps)) / args.steps
            for i, c in enumerate(calls)}

    # The roofline kernel: the slower of the two single-launch GEMM calls (forward:
    # Z = X.W with the fused bias + activation epilogue; dX = dP.W^T).
    dom = max(("forward_gemm", "dx_gemm"), key=lambda k: kern[k])
    gemm_flops = 2.0 * M * K * N
    achieved = gemm_flops / (kern[dom] * 1e-3) / 1e12
    peak = PEAK["f16" if half else "f32"]
    trec = traffic_record(args.config, dom)

    out = {
        "metric": "DenseBlock fwd+bwd TFLOP/s & % MFMA peak (fp16, B=8192, 4096→4096)",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if half else "f32",
        "data": "synthetic (seeded N(0,1) inputs, He-normal weights, N(0,1)*512 upstream gradient)",
        "config": {"workload": cfg["workload"], "M": M, "K": K, "N": N,
                   "pct_of_peak_step": round(100 * value / peak, 2), "wall_s": round(wall, 3)},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(achieved / peak, 4),
                     "traffic": trec["bytes_per_launch"] if trec else None,
                     "traffic_source": trec["source"] if trec else None, "kernel": dom,
                     "kernel_ms": {k: round(v, 4) for k, v in kern.items()}},
    }
    if not args.no_cpu:
        # the whole batch: about 10-20 s of the oracle on the host cores
        rows = args.cpu_rows or M
        out["cpu_baseline"] = cpu_baseline(cfg, rows)
    print(json.dumps(out), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
