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
  library_gemm  torch's bf16 matmul (hipBLASLt) timed on plain operands of
                the same three GEMM shapes, as a vendor-library reference
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
    import torch
    c = layer.get_coefficients()
    # a training step's optimizer updates the coefficients in place, which
    # advances their version; the layer keeps its packed operand per version,
    # so this makes every timed step re-pack as training does (with unchanged
    # coefficients the pack would be skipped: work left out of the step)
    torch.autograd.graph.increment_version(c)
    c.grad = None
    x.grad = None
    y = layer(x)
    y.backward(dy)


def _settle(layer, x, dy, seconds):
    """Untimed steps until `seconds` of wall time have passed: the GPU leaves
    its idle clock state and the caches reach the loop's steady state before
    the warm-up and timed steps.  Returns (steps, seconds) for the JSON line."""
    import torch
    n = 0
    t0 = time.perf_counter()
    while True:
        for _ in range(10):
            _step(layer, x, dy)
        n += 10
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= seconds:
            return n, time.perf_counter() - t0


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


def _library_gemms(iters=50):
    """torch's bf16 matmul (hipBLASLt) on plain operands of the three config-3
    contractions, for scale: the same (M, N, K) as the fused kernels, without
    the basis generation, the degree reduction or the epilogues they fuse.
    Operands in the (N, T) layout, the fastest of the three tried."""
    import torch
    shapes = {"fwd_gemm": (B, O, K), "dx_gemm": (B, I * DEG, O), "dc_gemm": (K, O, B)}
    out = {}
    for name, (m, n, k) in shapes.items():
        a = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        bt = torch.randn(n, k, device="cuda", dtype=torch.bfloat16)
        ms = _time_loop(lambda: a @ bt.t(), iters, 10)
        out[name] = {"m": m, "n": n, "k": k, "us": round(ms * 1e3, 1),
                     "tflops": round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 1)}
        del a, bt
    return out


SUITE = ("cfg1", "cfg2", "cfg4", "cfg5", "families", "fp64")
PEAK_FP64_TFLOPS = 78.6     # MI355X dense fp64


def _suite(only=SUITE, cpu=True):
    """Secondary BASELINE configs (1, 2, 4, 5) and the other bases; each takes well under a minute.
    With `cpu`, configs 1, 2, 4 and 5 carry the oracle's CPU timing on this host beside the GPU's."""
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
        # the 1000 README epochs issued by the library in one call (fit)
        # (the kernels are loaded and warm from the loops above)
        ex = kan_amd.ResidentExecutor([1, 1], [8], 100, compute="fp32", loss="mse",
                                      optimizer="adam", lr=0.01)
        ex.set_coeffs(0, m.cheby_coeffs.detach())
        fit_losses = []
        ms_fit = _time_loop(lambda: fit_losses.append(ex.fit(x1, y1, 1000)), 1, 0) / 1000
        ex.close()
        out["cfg1"] = {"workload": "ChebyKANLayer(1,1,8) sin(2 pi x), 100 pts, MSE+Adam, resident",
                       "us_per_step": ms_fit * 1e3, "steps": 1000,
                       "timing": "1000 steps issued by one ResidentExecutor.fit call "
                                 "(ckan_exec_steps): one single-workgroup launch runs them "
                                 "one after another, the state in LDS",
                       "final_loss": float(fit_losses[-1][-1].item()),
                       "us_per_step_python_step_loop": res1["eager"][0] * 1e3,
                       "us_per_step_hip_graph": res1["graph"][0] * 1e3}
        if cpu:
            cores = _cpu_threads()
            xc, yc = x1.cpu(), y1.cpu()
            torch.manual_seed(0)
            t, n, spent = _cpu_train([1, 1], [8], xc, yc, "mse", "adam", 0.01, 10, 2.0)
            out["cfg1"]["cpu_baseline"] = {
                "value": 1e6 * t, "unit": "us/step", "cores": cores, "kind": "port",
                "sample": f"the full config (100 points, Adam step), median of {n} steps after 1 warm-up "
                          f"({spent:.1f} s of CPU work)",
                "gpu_speedup": t * 1e6 / out["cfg1"]["us_per_step"]}

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
        ex = kan_amd.ResidentExecutor.from_sequential(seq, 256, compute="fp32", loss="ce",
                                                      optimizer="sgd", lr=0.01)
        ex.fit(x2, l2, 20)
        ms = _time_loop(lambda: ex.fit(x2, l2, 200), 1, 0) / 200
        ex.close()
        out["cfg2"] = {"workload": "784->64->10 deg 4 fp32 B=256, CE+SGD, resident",
                       "us_per_step": ms * 1e3, "samples_per_s": 256 / (ms * 1e-3),
                       "tflops": 2.618e8 / (ms * 1e-3) / 1e12,
                       "timing": "200 steps issued by one ResidentExecutor.fit call (ckan_exec_steps)",
                       "us_per_step_python_step_loop": res2["eager"] * 1e3,
                       "us_per_step_hip_graph": res2["graph"] * 1e3}
        if cpu:
            cores = _cpu_threads()
            torch.manual_seed(2)
            t, n, spent = _cpu_train([784, 64, 10], [4, 4], x2.cpu(), l2.cpu(), "ce", "sgd", 0.01, 10, 2.0)
            out["cfg2"]["cpu_baseline"] = {
                "value": 256 / t, "unit": "samples/s", "us_per_step": 1e6 * t, "cores": cores,
                "kind": "port",
                "sample": f"the full config (B=256, CE + SGD step), median of {n} steps after 1 warm-up "
                          f"({spent:.1f} s of CPU work)",
                "gpu_speedup": t * 1e3 / ms}

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
        if cpu:
            # one warm-up step on 4096 rows, then one timed step at the full 65536
            # rows (the per-step cost of 100 steps is 100 x this one)
            import torch.nn.functional as F
            from oracle import chebykan_oracle as orc
            cores = _cpu_threads()
            xc, tc4 = x4.cpu(), t4.cpu()
            torch.manual_seed(4)
            ps = [orc.init_coeffs(a, b, 16).requires_grad_(True)
                  for a, b in [(512, 512), (512, 512), (512, 512), (512, 64)]]
            opt = torch.optim.SGD(ps, lr=0.01)

            def step4(xs, ts):
                opt.zero_grad()
                F.mse_loss(orc.mlp_forward(xs, ps), ts).backward()
                opt.step()
            step4(xc[:4096], tc4[:4096])
            t0 = time.perf_counter()
            step4(xc, tc4)
            t = time.perf_counter() - t0
            del xc, tc4, ps, opt
            out["cfg4"]["cpu_baseline"] = {
                "value": 65536 / t, "unit": "samples/s", "s_per_step": t,
                "s_per_100_steps_extrapolated": 100 * t, "cores": cores, "kind": "port",
                "sample": "one full step (B=65536, MSE + SGD) after one 4096-row warm-up step; the "
                          "100-step figure is 100 x that step (extrapolated, not run)",
                "gpu_speedup": t * 1e3 / ms}

    if "cfg5" in only:
        # config 5: 2048->2048 deg 8, bf16 coefficients packed once, forward at B = 1, 16, 64.
        # "warm": the same packed coefficients every call (75.5 MB, inside the 256 MB
        # Infinity Cache after the first); "cold": calls rotate over NROT packed copies
        # whose forward operands total more than that cache, so each call streams its
        # coefficients from HBM.
        L = _lib.load()
        I5 = O5 = 2048
        NROT = 6
        g = torch.Generator().manual_seed(5)
        c5 = (torch.randn(I5, O5, 9, generator=g) / (I5 * 9)).bfloat16()
        res5 = {}
        packs = None
        for B5 in (1, 16, 64):
            d = _lib.make_desc(B5, I5, O5, 8, _lib.CKAN_COMPUTE_BF16, _lib.CKAN_DTYPE_BF16)
            st = _lib.stream_ptr(dev)
            if packs is None:  # the packed layout does not depend on the batch
                cdev = c5.to(dev)
                packs = []
                for _ in range(NROT):
                    pk = torch.empty(L.ckan_packed_bytes(d), dtype=torch.uint8, device=dev)
                    _lib.check(L.ckan_pack_coeffs(d, cdev.data_ptr(), pk.data_ptr(), st))
                    packs.append(pk)
                del cdev
            x5 = torch.randn(B5, I5, generator=g).to(dev)
            y5 = torch.empty(B5, O5, device=dev)
            t5 = torch.empty(L.ckan_tcache_elems(d), device=dev)
            wsb = L.ckan_fwd_workspace_bytes(d)
            ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device=dev)
            k = [0]

            def fwd(rotate):
                pk = packs[k[0] % NROT] if rotate else packs[0]
                k[0] += 1
                _lib.check(L.ckan_forward(d, x5.data_ptr(), pk.data_ptr(), y5.data_ptr(),
                                          t5.data_ptr(), ws.data_ptr(), wsb, st))
            alg_bytes = I5 * O5 * 9 * 2 + B5 * I5 * 4 + B5 * O5 * 4
            ent = {"alg_bytes": alg_bytes}
            for mode, rot in (("warm", False), ("cold", True)):
                ms = _time_loop(lambda: fwd(rot), 300, 30)
                _lib.profile_report()
                _lib.profile_enable(True)
                for _ in range(60):
                    fwd(rot)
                torch.cuda.synchronize()
                _lib.profile_enable(False)
                rep = _lib.profile_report()
                gemm_ms = rep["fwd_gemm"][1] / rep["fwd_gemm"][0]
                ent[mode] = {"us_forward": ms * 1e3, "us_gemm": gemm_ms * 1e3,
                             "gemm_GBps": alg_bytes / (gemm_ms * 1e-3) / 1e9,
                             "frac_hbm_peak": alg_bytes / (gemm_ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
                             "forward_GBps": alg_bytes / (ms * 1e-3) / 1e9}
            # the drop-in layer: ChebyKANLayer(2048, 2048, 8) with bf16 coefficients,
            # called under no_grad; its packed operands are cached per coefficient
            # version, so each call runs the forward alone (cold: NROT layers rotated)
            layers = []
            for _ in range(NROT):
                m = kan_amd.ChebyKANLayer(I5, O5, 8, compute="bf16").to(dev)
                m.cheby_coeffs.data = c5.to(dev)
                layers.append(m)
            kk = [0]

            def lfwd():
                m = layers[kk[0] % NROT]
                kk[0] += 1
                return m(x5)
            with torch.no_grad():
                for m in layers:
                    m(x5)  # packs once
                torch.cuda.synchronize()
                ms_layer = _time_loop(lfwd, 300, 30)
                y_layer = layers[0](x5)
                torch.cuda.synchronize()
            assert torch.equal(y_layer, y5), "layer and raw forward disagree"
            ent["cold"]["us_layer_forward"] = ms_layer * 1e3
            ent["cold"]["layer_over_raw"] = ms_layer * 1e3 / ent["cold"]["us_forward"]
            del layers
            if cpu:
                from oracle import chebykan_oracle as orc
                cores = _cpu_threads()
                xc, cc = x5.cpu(), c5.float()
                t, n, spent = _cpu_median(lambda: orc.layer_forward(xc, cc), 3, 1.5, 50)
                ent["cpu_baseline"] = {
                    "value": B5 / t, "unit": "samples/s", "ms_per_forward": 1e3 * t, "cores": cores,
                    "kind": "port",
                    "sample": f"the full forward at B={B5} (fp32 math on the bf16-rounded coefficients), "
                              f"median of {n} calls after 1 warm-up ({spent:.1f} s of CPU work)",
                    "gpu_speedup_cold": t * 1e3 / ent["cold"]["us_forward"] * 1e3}
            res5[f"B{B5}"] = ent
        del packs
        out["cfg5"] = {"workload": "ChebyKANLayer(2048,2048,8) inference, bf16 coefficients (packed once); "
                                   f"warm = one packed copy, cold = {NROT} copies rotated (forward "
                                   "operands above the 256 MB Infinity Cache); us_layer_forward = "
                                   "the drop-in module called under no_grad (its packed operands "
                                   f"cached per coefficient version), {NROT} modules rotated",
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
            # untimed steps first, as for the headline: the figure is the steady
            # state, not the clock ramp after the previous entry's idle gaps
            _settle(layer, xf, dyf, 0.5)
            ms = _time_gpu(layer, xf, dyf, 30, 10)
            kern = _kernel_breakdown(layer, xf, dyf, 10)
            fam[name] = {"ms_per_step": ms, "samples_per_s": B / (ms * 1e-3),
                         "tflops": STEP_FLOP / (ms * 1e-3) / 1e12,
                         # the pack launch also computes tanh(x) where the layout allows
                         "pack_ms": kern.get("pack_tanh", kern.get("pack", {})).get("avg_ms"),
                         # dC' M^T: in the dC launch's epilogue where one launch writes
                         # the whole gradient (no separate map launch, None here)
                         "dc_gemm_ms": kern["dc_gemm"]["avg_ms"],
                         "coeff_from_cheb_ms": kern.get("coeff_from_cheb", {}).get("avg_ms")}
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


def _cpu_info():
    """The host the CPU baselines ran on: nproc, the CPUs this process may use,
    the threads torch runs with, and lscpu's identification of the part."""
    import subprocess
    import torch
    info = {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "threads": torch.get_num_threads()}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            key = key.strip()
            if key in ("Model name", "CPU family", "Model", "Stepping", "Socket(s)",
                       "Core(s) per socket", "Thread(s) per core", "Vendor ID"):
                info["lscpu " + key] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def _cpu_threads():
    import torch
    torch.set_num_threads(len(os.sched_getaffinity(0)) or 1)
    return torch.get_num_threads()


def _cpu_median(fn, min_reps, min_seconds, max_reps=1000):
    """One warm-up call, then at least `min_reps` timed calls and about
    `min_seconds` of work; returns (median seconds, calls timed, seconds spent)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t_start < min_seconds and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times), time.perf_counter() - t_start


def _cpu_baseline(sample_rows: int, reps: int):
    """Config 3 on the CPU: the oracle's op-for-op restatement of the reference
    layer (forward + autograd backward, dx and dC) on a sample of the rows."""
    import torch
    from oracle import chebykan_oracle as orc
    cores = _cpu_threads()
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(sample_rows, I, generator=g)
    c = torch.randn(I, O, DEG + 1, generator=g) / (I * (DEG + 1))
    dy = torch.randn(sample_rows, O, generator=g)
    t, n, spent = _cpu_median(lambda: orc.layer_forward_backward(x, c, dy), reps, 10.0)
    return {
        "value": sample_rows / t,
        "unit": "samples/s",
        "cores": cores,
        "kind": "port",
        "host": _cpu_info(),
        "sample": (f"config-3 layer (1024->1024, deg 8) fwd+bwd(dx,dC) on {sample_rows} of the "
                   f"{B} rows, fp32 torch CPU op-for-op restatement of "
                   f"kan/basis/chebyshev.py:78,92-101,130-145 + autograd; median of {n} "
                   f"steps after 1 warm-up ({t * 1e3:.1f} ms/step, {spent:.1f} s of CPU work)"),
    }


def _cpu_train(widths, degrees, x, target, loss, optimizer, lr, min_reps, min_seconds):
    """Median CPU time of one reference training step (README.md:61-69 over a
    KANSequential): zero_grad, the oracle's forward, torch's loss, backward and
    torch.optim's step."""
    import torch
    import torch.nn.functional as F
    from oracle import chebykan_oracle as orc
    ps = [orc.init_coeffs(widths[l], widths[l + 1], degrees[l]).requires_grad_(True)
          for l in range(len(degrees))]
    opt = (torch.optim.Adam if optimizer == "adam" else torch.optim.SGD)(ps, lr=lr)
    lossf = F.mse_loss if loss == "mse" else F.cross_entropy

    def step():
        opt.zero_grad()
        lossf(orc.mlp_forward(x, ps), target).backward()
        opt.step()
    return _cpu_median(step, min_reps, min_seconds)


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
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-s", type=float, default=1.0,
                    help="untimed steps for this many seconds before the warm-up (0: none); "
                         "reported in the JSON line")
    ap.add_argument("--compute", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--cpu-rows", type=int, default=B,
                    help="config-3 rows in the CPU baseline's step (default: all of them)")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-fp32", action="store_true")
    ap.add_argument("--no-suite", action="store_true", help="skip configs 1, 2, 4, 5")
    ap.add_argument("--suite-only", default=",".join(SUITE),
                    help="comma list of suite entries to run (default: all of %s)" % (SUITE,))
    ap.add_argument("--no-library", action="store_true",
                    help="skip the hipBLASLt reference GEMMs at the same shapes")
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

    settle_steps, settle_s = _settle(layer, x, dy, args.settle_s) if args.settle_s > 0 else (0, 0.0)
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
    if not args.no_library and args.compute == "bf16":
        extra["library_gemm"] = _library_gemms()

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
        "settle": {"steps": settle_steps, "seconds": round(settle_s, 3),
                   "note": "untimed steps run before the warm-up steps, so the timed steps "
                           "see the GPU's steady-state clocks rather than its idle state"},
        "kernels_avg_ms": {k: round(v["avg_ms"], 5) for k, v in kernels.items()},
        **extra,
    }
    if not args.no_suite:
        only = tuple(n for n in args.suite_only.split(",") if n)
        unknown = set(only) - set(SUITE)
        if unknown:
            ap.error(f"unknown suite entries {sorted(unknown)}")
        out["configs"] = _suite(only, cpu=not args.no_cpu)
    if not args.no_cpu:
        out["cpu_baseline"] = _cpu_baseline(args.cpu_rows, args.cpu_reps)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
