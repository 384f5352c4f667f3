"""Headline benchmark: fused ChebyKAN forward+backward on one MI355X.

Workload (the north-star target): one
ChebyKANLayer(1024, 1024, degree=8), batch 8192, x ~ N(0,1),
C ~ N(0, 1/(1024*9)), upstream gradient dy ~ N(0,1), x.requires_grad=True.
One step = coefficient pack + forward + backward (dx and dC), driven
through the drop-in layer API (autograd), all inputs resident in HBM.
Compute: bf16 MFMA with fp32 accumulation (the fp32-MFMA variant is
reported alongside).

Prints ONE JSON line.  Besides the driver contract fields it carries
  roofline      for the dominant kernel, from HIP events recorded by the
                library on the launch stream over a second timed pass
  cpu_baseline  the oracle's op-for-op torch restatement of the reference
                path, timed on this host's cores on a bounded sample
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_FP32_TFLOPS = 157.3    # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0

B, I, O, DEG = 8192, 1024, 1024, 8
K = I * (DEG + 1)
GEMM_FLOP = 2.0 * B * K * O          # one contraction (fwd, dX or dC)
STEP_FLOP = 3.0 * GEMM_FLOP          # x requires grad: fwd + dX + dC


def _step(layer, x, dy):
    layer.cheby_coeffs.grad = None
    x.grad = None
    y = layer(x)
    y.backward(dy)


def _time_gpu(layer, x, dy, steps, warmup):
    import torch
    for _ in range(warmup):
        _step(layer, x, dy)
    torch.cuda.synchronize()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        _step(layer, x, dy)
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def _kernel_breakdown(layer, x, dy, steps):
    """Per-kernel average durations from the library's HIP events."""
    import torch
    from kan_amd import _lib
    torch.cuda.synchronize()
    _lib.profile_report()  # clear
    _lib.profile_enable(True)
    for _ in range(steps):
        _step(layer, x, dy)
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    rep = _lib.profile_report()
    return {k: {"launches": c, "avg_ms": ms / c} for k, (c, ms) in rep.items()}


def _cpu_baseline(sample_rows: int, reps: int):
    import torch
    from oracle import chebykan_oracle as orc
    torch.set_num_threads(os.cpu_count() or 1)
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(sample_rows, I, generator=g)
    c = torch.randn(I, O, DEG + 1, generator=g) / (I * (DEG + 1))
    dy = torch.randn(sample_rows, O, generator=g)
    orc.layer_forward_backward(x, c, dy)  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        orc.layer_forward_backward(x, c, dy)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    return {
        "value": sample_rows / t,
        "unit": "samples/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"config-3 layer (1024->1024, deg 8) fwd+bwd(dx,dC) on {sample_rows} of the "
                   f"8192 rows, fp32 torch CPU op-for-op restatement of "
                   f"kan/basis/chebyshev.py:78,92-101,130-145 + autograd; median of {reps} "
                   f"after 1 warm-up ({t * 1e3:.1f} ms/step)"),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--compute", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fp32", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU; --gpus {args.gpus} is not "
              f"supported (no multi-GPU path).", file=sys.stderr)
        sys.exit(2)

    import torch
    import kan_amd

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    layer = kan_amd.ChebyKANLayer(I, O, DEG, compute=args.compute)
    g = torch.Generator().manual_seed(42)
    with torch.no_grad():
        layer.cheby_coeffs.copy_(torch.randn(I, O, DEG + 1, generator=g) / (I * (DEG + 1)))
    layer = layer.to(dev)
    x = torch.randn(B, I, generator=g).to(dev).requires_grad_(True)
    dy = torch.randn(B, O, generator=g).to(dev)

    ms = _time_gpu(layer, x, dy, args.steps, args.warmup)
    kernels = _kernel_breakdown(layer, x, dy, args.steps)

    peak = PEAK_BF16_TFLOPS if args.compute == "bf16" else PEAK_FP32_TFLOPS
    gemms = {k: v for k, v in kernels.items() if k.endswith("_gemm")}
    dom = max(gemms, key=lambda k: gemms[k]["avg_ms"])
    achieved = GEMM_FLOP / (gemms[dom]["avg_ms"] * 1e-3) / 1e12
    tflops = STEP_FLOP / (ms * 1e-3) / 1e12

    extra = {}
    if not args.no_fp32 and args.compute == "bf16":
        layer.compute = "fp32"
        ms32 = _time_gpu(layer, x, dy, max(3, args.steps // 4), 2)
        layer.compute = args.compute
        t32 = STEP_FLOP / (ms32 * 1e-3) / 1e12
        extra["fp32_variant"] = {"ms_per_step": ms32, "samples_per_s": B / (ms32 * 1e-3),
                                 "tflops": t32, "frac_fp32_peak": t32 / PEAK_FP32_TFLOPS}

    out = {
        "metric": "fused ChebyKAN fwd+bwd samples/s & TFLOP/s (% MFMA peak), 1 MI355X",
        "value": B / (ms * 1e-3),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.compute,
        "data": "synthetic",
        "config": {
            "workload": (f"ChebyKANLayer(1024, 1024, degree=8), batch 8192, pack+fwd+bwd(dx,dC), "
                         f"{args.compute} MFMA fp32-accumulate (BASELINE configs[2])"),
            "batch": B, "in_dim": I, "out_dim": O, "degree": DEG,
        },
        "tflops": tflops,
        "frac_of_peak": tflops / peak,
        "roofline": {
            "bound": "mfma",
            "kernel": dom,
            "achieved": achieved,
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": achieved / peak,
            "traffic": None,
        },
        "kernels_avg_ms": {k: round(v["avg_ms"], 5) for k, v in kernels.items()},
        **extra,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = _cpu_baseline(args.cpu_rows, args.cpu_reps)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
