"""Fused SGD and Adam steps for device parameters.

Both follow torch.optim's single-tensor update order (torch/optim/sgd.py,
torch/optim/adam.py), which the reference's training loop uses
(README.md:58-66), and run as one HIP kernel per parameter tensor.  Only
fp32 contiguous ROCm-device parameters are accepted.
"""
from __future__ import annotations

from typing import Iterable, Tuple

import torch
from torch.autograd.graph import increment_version

from . import _lib


def _check_param(p: torch.Tensor) -> None:
    if not p.is_cuda or p.dtype != torch.float32 or not p.is_contiguous():
        raise RuntimeError("kan_amd optimizers need fp32 contiguous parameters on a ROCm device")


class SGD(torch.optim.Optimizer):
    """p -= lr * (g + weight_decay * p); no momentum."""

    def __init__(self, params: Iterable, lr: float = 1e-3, weight_decay: float = 0.0):
        if lr < 0.0:
            raise ValueError(f"Invalid learning rate: {lr}")
        super().__init__(params, dict(lr=lr, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        lib = _lib.load()
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                _check_param(p)
                g = p.grad.contiguous()
                _lib.check(lib.ckan_sgd_step(p.data_ptr(), g.data_ptr(), p.numel(),
                                             float(group["lr"]), float(group["weight_decay"]),
                                             _lib.stream_ptr(p.device)))
                # the kernel wrote p through its pointer: advance its version as a
                # torch in-place op would (the layers' packed-operand caches key on it)
                increment_version(p)
        return loss


class Adam(torch.optim.Optimizer):
    """Adam (no amsgrad) with torch's defaults betas=(0.9, 0.999), eps=1e-8."""

    def __init__(self, params: Iterable, lr: float = 1e-3, betas: Tuple[float, float] = (0.9, 0.999),
                 eps: float = 1e-8, weight_decay: float = 0.0):
        if lr < 0.0:
            raise ValueError(f"Invalid learning rate: {lr}")
        if not 0.0 <= betas[0] < 1.0 or not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid betas: {betas}")
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        lib = _lib.load()
        for group in self.param_groups:
            b1, b2 = group["betas"]
            for p in group["params"]:
                if p.grad is None:
                    continue
                _check_param(p)
                st = self.state[p]
                if not st:
                    # torch.optim.Adam keeps the count as a float32 CPU tensor, so
                    # state_dicts load both ways
                    st["step"] = torch.tensor(0.0, dtype=torch.float32)
                    st["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                    st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                if not torch.is_tensor(st["step"]):
                    st["step"] = torch.tensor(float(st["step"]), dtype=torch.float32)
                for k in ("exp_avg", "exp_avg_sq"):
                    if st[k].device != p.device or not st[k].is_contiguous():
                        st[k] = st[k].to(p.device, torch.float32).contiguous()
                # rebind rather than add in place: a loaded state_dict may share
                # this tensor with the optimizer it came from
                st["step"] = st["step"] + 1
                step = int(st["step"].item())
                g = p.grad.contiguous()
                _lib.check(lib.ckan_adam_step(
                    p.data_ptr(), g.data_ptr(), st["exp_avg"].data_ptr(),
                    st["exp_avg_sq"].data_ptr(), p.numel(), step, float(group["lr"]),
                    float(b1), float(b2), float(group["eps"]), float(group["weight_decay"]),
                    _lib.stream_ptr(p.device)))
                increment_version(p)  # written through its pointer (see SGD.step)
        return loss
