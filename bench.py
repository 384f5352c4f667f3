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
    layer.get_coefficients().grad = None
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


def _time_loop(fn, iters, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


SUITE = ("cfg1", "cfg2", "cfg4", "cfg5", "families", "fp64")
PEAK_FP64_TFLOPS = 78.6     # MI355X dense fp64


def _suite(only=SUITE):
    """Secondary BASELINE configs (1, 2, 4, 5) and the other bases; each takes well under a minute."""
    import ctypes
    import math
    import torch
    import kan_amd
    from kan_amd import _lib
    dev = torch.device("cuda:0")
    out = {}

    if "cfg1" in only:
        # config 1: ChebyKANLayer(1,1,8), 100 points, MSE + Adam lr 0.01, 1000 steps (README.md:42-73)
        torch.manual_seed(0)
        m = kan_amd.ChebyKANLayer(1, 1, 8)
        x1 = torch.linspace(-1, 1, 100).reshape(-1, 1).to(dev)
        y1 = torch.sin(2 * math.pi * x1)
        res1 = {}
        for graph in (False, True):
            ex = kan_amd.ResidentExecutor([1, 1], [8], 100, compute="fp32", loss="mse",
                                          optimizer="adam", lr=0.01, use_graph=graph)
            ex.set_coeffs(0, m.cheby_coeffs.detach())
            ms = _time_loop(lambda: ex.step(x1, y1), 1000, 0)
            res1["graph" if graph else "eager"] = (ms, float(ex.step(x1, y1).item()))
            ex.close()
        out["cfg1"] = {"workload": "ChebyKANLayer(1,1,8) sin(2 pi x), 100 pts, MSE+Adam, resident, eager launches",
                       "us_per_step": res1["eager"][0] * 1e3, "steps": 1000,
                       "final_loss": res1["eager"][1],
                       "us_per_step_hip_graph": res1["graph"][0] * 1e3}

    if "cfg2" in only:
        # config 2: 784->64->10, deg 4, fp32, B=256, CE + SGD lr 0.01
        g = torch.Generator().manual_seed(2)
        x2 = (torch.rand(256, 784, generator=g) * (torch.rand(256, 784, generator=g) >= 0.8).float()).to(dev)
        l2 = torch.randint(0, 10, (256,), generator=g).to(dev)
        torch.manual_seed(2)
        seq = kan_amd.KANSequential(kan_amd.ChebyKANLayer(784, 64, 4), kan_amd.ChebyKANLayer(64, 10, 4))
        res2 = {}
        for graph in (False, True):
            ex = kan_amd.ResidentExecutor.from_sequential(seq, 256, compute="fp32", loss="ce",
                                                          optimizer="sgd", lr=0.01, use_graph=graph)
            res2["graph" if graph else "eager"] = _time_loop(lambda: ex.step(x2, l2), 200, 20)
            ex.close()
        ms = res2["eager"]
        out["cfg2"] = {"workload": "784->64->10 deg 4 fp32 B=256, CE+SGD, resident, eager launches",
                       "us_per_step": ms * 1e3, "samples_per_s": 256 / (ms * 1e-3),
                       "tflops": 2.618e8 / (ms * 1e-3) / 1e12,
                       "us_per_step_hip_graph": res2["graph"] * 1e3}

    if "cfg4" in only:
        # config 4: 512->512->512->512->64, deg 16, B=65536, fp32 masters + bf16 compute, MSE + SGD, 100 steps
        g = torch.Generator().manual_seed(4)
        x4 = (torch.rand(65536, 512, generator=g) * 6 - 3).to(dev)
        W = (torch.randn(512, 64, generator=g) / math.sqrt(512)).to(dev)
        t4 = x4 @ W + 0.1 * torch.randn(65536, 64, generator=g).to(dev)
        torch.manual_seed(4)
        seq = kan_amd.KANSequential(*[kan_amd.ChebyKANLayer(a, b, 16)
                                      for a, b in [(512, 512), (512, 512), (512, 512), (512, 64)]])
        ex = kan_amd.ResidentExecutor.from_sequential(seq, 65536, compute="bf16", loss="mse",
                                                      optimizer="sgd", lr=0.01)
        ms = _time_loop(lambda: ex.step(x4, t4), 100, 3)
        out["cfg4"] = {"workload": "512->512->512->512->64 deg 16 B=65536 bf16 MFMA, fp32 masters, MSE+SGD, resident",
                       "ms_per_step": ms, "samples_per_s": 65536 / (ms * 1e-3),
                       "tflops": 4.8920e12 / (ms * 1e-3) / 1e12,
                       "frac_bf16_peak": 4.8920e12 / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS,
                       "final_loss": float(ex.step(x4, t4).item())}
        ex.close()

    if "cfg5" in only:
        # config 5: 2048->2048 deg 8, bf16 coefficients packed once, forward at B = 1, 16, 64
        L = _lib.load()
        I5 = O5 = 2048
        g = torch.Generator().manual_seed(5)
        c5 = (torch.randn(I5, O5, 9, generator=g) / (I5 * 9)).bfloat16().to(dev)
        res5 = {}
        for B5 in (1, 16, 64):
            d = _lib.make_desc(B5, I5, O5, 8, _lib.CKAN_COMPUTE_BF16, _lib.CKAN_DTYPE_BF16)
            st = _lib.stream_ptr(dev)
            packed = torch.empty(L.ckan_packed_bytes(d), dtype=torch.uint8, device=dev)
            _lib.check(L.ckan_pack_coeffs(d, c5.data_ptr(), packed.data_ptr(), st))
            x5 = torch.randn(B5, I5, generator=g).to(dev)
            y5 = torch.empty(B5, O5, device=dev)
            t5 = torch.empty(L.ckan_tcache_elems(d), device=dev)
            wsb = L.ckan_fwd_workspace_bytes(d)
            ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
            fwd = lambda: _lib.check(L.ckan_forward(d, x5.data_ptr(), packed.data_ptr(), y5.data_ptr(),
                                                    t5.data_ptr(), ws.data_ptr(), wsb, st))
            ms = _time_loop(fwd, 200, 20)
            _lib.profile_report()
            _lib.profile_enable(True)
            for _ in range(50):
                fwd()
            torch.cuda.synchronize()
            _lib.profile_enable(False)
            rep = _lib.profile_report()
            gemm_ms = rep["fwd_gemm"][1] / rep["fwd_gemm"][0]
            alg_bytes = I5 * O5 * 9 * 2 + B5 * I5 * 4 + B5 * O5 * 4
            res5[f"B{B5}"] = {"us_forward": ms * 1e3, "us_gemm": gemm_ms * 1e3,
                              "gemm_GBps": alg_bytes / (gemm_ms * 1e-3) / 1e9,
                              "frac_hbm_peak": alg_bytes / (gemm_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                              "alg_bytes": alg_bytes}
        out["cfg5"] = {"workload": "ChebyKANLayer(2048,2048,8) inference, bf16 coefficients (packed once)",
                       **res5}

    if "families" in only:
        # the Jacobi / Hermite layers at the config-3 shape: same kernels plus the
        # change of basis in the pack and the dC back-transform
        fam = {}
        g = torch.Generator().manual_seed(6)
        xf = torch.randn(B, I, generator=g).to(dev).requires_grad_(True)
        dyf = torch.randn(B, O, generator=g).to(dev)
        for name, make in (("JacobiKANLayer(alpha=0.5,beta=0.5)",
                            lambda: kan_amd.JacobiKANLayer(I, O, DEG, alpha=0.5, beta=0.5, compute="bf16")),
                           ("HermiteKANLayer(physicist)",
                            lambda: kan_amd.HermiteKANLayer(I, O, DEG, compute="bf16"))):
            torch.manual_seed(6)
            layer = make().to(dev)
            ms = _time_gpu(layer, xf, dyf, 30, 10)
            kern = _kernel_breakdown(layer, xf, dyf, 10)
            fam[name] = {"ms_per_step": ms, "samples_per_s": B / (ms * 1e-3),
                         "tflops": STEP_FLOP / (ms * 1e-3) / 1e12,
                         "pack_ms": kern["pack"]["avg_ms"],
                         "coeff_from_cheb_ms": kern["coeff_from_cheb"]["avg_ms"]}
        out["families_cfg3_shape"] = {"workload": "1024->1024 deg 8, B=8192, bf16 MFMA, pack+fwd+bwd",
                                      **fam}


    if "fp64" in only:
        # the layer with fp64 parameters (the reference computes in fp64 then), config-3 shape
        torch.manual_seed(7)
        layer = kan_amd.ChebyKANLayer(I, O, DEG).double().to(dev)
        g = torch.Generator().manual_seed(7)
        x64 = torch.randn(B, I, generator=g, dtype=torch.float64).to(dev).requires_grad_(True)
        dy64 = torch.randn(B, O, generator=g, dtype=torch.float64).to(dev)
        ms = _time_gpu(layer, x64, dy64, 5, 2)
        kern = _kernel_breakdown(layer, x64, dy64, 3)
        t = STEP_FLOP / (ms * 1e-3) / 1e12
        out["fp64_cfg3_shape"] = {"workload": "ChebyKANLayer(1024,1024,8).double(), B=8192, fwd+bwd in fp64",
                                  "ms_per_step": ms, "samples_per_s": B / (ms * 1e-3), "tflops": t,
                                  "frac_fp64_peak": t / PEAK_FP64_TFLOPS,
                                  "fwd_ms": kern["fwd_f64"]["avg_ms"], "bwd_ms": kern["bwd_f64"]["avg_ms"]}
    return out


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
    t_start = time.perf_counter()
    # at least `reps` steps, and about 10 s of CPU work in all
    while len(times) < reps or time.perf_counter() - t_start < 10.0:
        t0 = time.perf_counter()
        orc.layer_forward_backward(x, c, dy)
        times.append(time.perf_counter() - t0)
        if len(times) >= 1000:
            break
    t = statistics.median(times)
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": sample_rows / t,
        "unit": "samples/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "cpu_model": model,
        "sample": (f"config-3 layer (1024->1024, deg 8) fwd+bwd(dx,dC) on {sample_rows} of the "
                   f"8192 rows, fp32 torch CPU op-for-op restatement of "
                   f"kan/basis/chebyshev.py:78,92-101,130-145 + autograd; median of {len(times)} "
                   f"steps after 1 warm-up ({t * 1e3:.1f} ms/step, "
                   f"{time.perf_counter() - t_start:.1f} s of CPU work)"),
    }


def _traffic(kernel: str, compute: str):
    """HBM bytes per launch of `kernel` from the committed counter summary
    (rocprofv3 FETCH_SIZE and WRITE_SIZE passes over this benchmark, each
    scaled by the same counter's reading on a plain copy of known size), or
    None when no summary for this kernel and precision is present."""
    path = os.path.join(ROOT, "profiles", f"traffic_cfg3_{compute}.json")
    try:
        with open(path) as f:
            data = json.load(f)
        return data["kernels"][kernel]["hbm_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--compute", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--cpu-rows", type=int, default=1024)
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fp32", action="store_true")
    ap.add_argument("--no-suite", action="store_true", help="skip configs 1, 2, 4, 5")
    ap.add_argument("--suite-only", default=",".join(SUITE),
                    help="comma list of suite entries to run (default: all of %s)" % (SUITE,))
    ap.add_argument("--copy-calib-mib", type=int, default=0,
                    help="run a plain device copy of this many MiB first (counter calibration)")
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

    if args.copy_calib_mib > 0:
        # a plain elementwise copy of known size: reads and writes N MiB once
        n = args.copy_calib_mib * (1 << 20) // 4
        src = torch.rand(n, device=dev)
        dst = torch.empty_like(src)
        torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst

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
            "traffic": _traffic(dom, args.compute),
        },
        "kernels_avg_ms": {k: round(v["avg_ms"], 5) for k, v in kernels.items()},
        **extra,
    }
    if not args.no_suite:
        only = tuple(n for n in args.suite_only.split(",") if n)
        unknown = set(only) - set(SUITE)
        if unknown:
            ap.error(f"unknown suite entries {sorted(unknown)}")
        out["configs"] = _suite(only)
    if not args.no_cpu:
        out["cpu_baseline"] = _cpu_baseline(args.cpu_rows, args.cpu_reps)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
