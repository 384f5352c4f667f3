"""CPU oracle: a restatement of the reference ChebyKAN hot path.

TEST INFRASTRUCTURE ONLY.  This module is the checker for the HIP path in
``kan_amd`` and the timed CPU baseline of ``bench.py``.  Nothing in the
product imports it.

Two independent restatements live here:

* an op-for-op torch (CPU) restatement of the reference layer, using the same
  aten ops the reference calls, so its fp32 rounding is the reference's:
    - ``normalize_input``      follows kan/basis/chebyshev.py:68-78
    - ``basis_closed_form``    follows kan/basis/chebyshev.py:119-145 (default)
    - ``basis_recurrence``     follows kan/basis/chebyshev.py:147-172
    - ``layer_forward``        follows kan/layers/chebykan.py:53-67 and
                               kan/basis/chebyshev.py:80-101
    - ``layer_forward_backward`` is torch autograd through that restatement,
                               which is what the reference's backward is
    - ``init_coeffs``          follows kan/layers/chebykan.py:46-51
    - ``adam_step``/``sgd_step`` restate torch.optim.Adam / SGD single-tensor
                               updates (torch/optim/adam.py, sgd.py), which
                               the reference's README loop uses (README.md:58-66)
* an fp64 numpy restatement from the mathematics (``*_fp64``), used to pin the
  torch restatement: T_n(cos th) = cos(n th), the explicit power-sum form of
  T_n, brute-force triple loops, and the closed-form input derivative
  d/dx sum_d g_d T_d(tanh x) = sum_d g_d d U_{d-1}(tanh x) (1 - tanh^2 x).

Parity status: every function above is pinned by a check in
tests/test_oracle.py (closed forms, special values, brute force, finite
differences, torch.optim itself).  The reference ships no golden vectors.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn.functional as F

__all__ = [
    "normalize_input", "basis_closed_form", "basis_recurrence", "layer_forward",
    "layer_forward_backward", "init_coeffs", "adam_step", "sgd_step",
    "cheb_T_fp64", "cheb_T_powersum_fp64", "cheb_U_fp64", "forward_fp64",
    "backward_fp64", "forward_bruteforce", "mlp_forward", "train_steps", "round_bf16_ste",
    "SATURATION_X",
]

# Smallest |x| for which fp32 tanh(x) rounds to exactly +-1.  At and beyond it
# the reference's closed-form backward produces NaN (acos'(+-1) = -inf times 0).
SATURATION_X = 9.0108


# ---------------------------------------------------------------------------
# op-for-op torch restatement of the reference (CPU)
# ---------------------------------------------------------------------------

def normalize_input(x: torch.Tensor) -> torch.Tensor:
    """t = tanh(x)  (kan/basis/chebyshev.py:78)."""
    return torch.tanh(x)


def basis_closed_form(t: torch.Tensor, degree: int) -> torch.Tensor:
    """T_n(t) = cos(n * acos(clamp(t, -1, 1))), n = 0..degree.

    kan/basis/chebyshev.py:130-145; the arange is fp32 (chebyshev.py:39).
    ``t`` is [B, in]; returns [B, in, degree+1].
    """
    b, i = t.shape
    t3 = t.view(b, i, 1)
    arccos_x = torch.acos(torch.clamp(t3, -1.0, 1.0))
    arange = torch.arange(0, degree + 1, dtype=torch.float32)
    return torch.cos(arccos_x * arange)


def basis_recurrence(t: torch.Tensor, degree: int) -> torch.Tensor:
    """T_0 = 1, T_1 = t, T_{n+1} = 2 t T_n - T_{n-1}  (chebyshev.py:157-172)."""
    b, i = t.shape
    out = torch.ones(b, i, degree + 1, dtype=t.dtype)
    if degree > 0:
        out[:, :, 1] = t
        for n in range(2, degree + 1):
            out[:, :, n] = 2 * t * out[:, :, n - 1] - out[:, :, n - 2]
    return out


def layer_forward(x: torch.Tensor, coeffs: torch.Tensor,
                  use_recurrence: bool = False) -> torch.Tensor:
    """y[b,o] = sum_{i,d} T_d(tanh x[b,i]) C[i,o,d].

    kan/layers/chebykan.py:64-67 -> kan/basis/chebyshev.py:92-101.
    """
    in_dim = coeffs.shape[0]
    x = x.view(-1, in_dim)
    t = normalize_input(x)
    deg = coeffs.shape[2] - 1
    basis = basis_recurrence(t, deg) if use_recurrence else basis_closed_form(t, deg)
    return torch.einsum("bid,iod->bo", basis, coeffs)


def layer_forward_backward(x: torch.Tensor, coeffs: torch.Tensor, dy: torch.Tensor,
                           need_dx: bool = True, need_dc: bool = True,
                           use_recurrence: bool = False):
    """Forward plus torch autograd backward of the restatement.

    Returns (y, dx or None, dC or None).  This is exactly how the reference
    obtains its gradients: it has no hand-written backward.
    """
    x = x.detach().clone().requires_grad_(need_dx)
    c = coeffs.detach().clone().requires_grad_(need_dc)
    y = layer_forward(x, c, use_recurrence)
    y.backward(dy)
    return y.detach(), (x.grad if need_dx else None), (c.grad if need_dc else None)


def init_coeffs(input_dim: int, output_dim: int, degree: int,
                init_scale: Optional[float] = None, seed: Optional[int] = None) -> torch.Tensor:
    """cheby_coeffs ~ N(0, std=init_scale or 1/(in*(deg+1))) on the CPU generator.

    kan/layers/chebykan.py:47-51 (note: ``or``, so init_scale=0.0 falls back).
    """
    if seed is not None:
        torch.manual_seed(seed)
    init_scale = init_scale or 1.0 / (input_dim * (degree + 1))
    c = torch.empty(input_dim, output_dim, degree + 1)
    torch.nn.init.normal_(c, mean=0.0, std=init_scale)
    return c


def adam_step(p: torch.Tensor, g: torch.Tensor, m: torch.Tensor, v: torch.Tensor,
              step: int, lr: float = 1e-3, betas: Tuple[float, float] = (0.9, 0.999),
              eps: float = 1e-8, weight_decay: float = 0.0) -> None:
    """In-place Adam update in torch's single-tensor order (torch/optim/adam.py).

    ``step`` is the step count after increment (1 on the first call).
    """
    beta1, beta2 = betas
    if weight_decay != 0:
        g = g.add(p, alpha=weight_decay)
    m.lerp_(g, 1 - beta1)
    v.mul_(beta2).addcmul_(g, g, value=1 - beta2)
    bias_correction1 = 1 - beta1 ** step
    bias_correction2 = 1 - beta2 ** step
    step_size = lr / bias_correction1
    denom = (v.sqrt() / (bias_correction2 ** 0.5)).add_(eps)
    p.addcdiv_(m, denom, value=-step_size)


def sgd_step(p: torch.Tensor, g: torch.Tensor, lr: float, weight_decay: float = 0.0) -> None:
    """p -= lr * g  (torch/optim/sgd.py, no momentum)."""
    if weight_decay != 0:
        g = g.add(p, alpha=weight_decay)
    p.add_(g, alpha=-lr)


def round_bf16_ste(c: torch.Tensor) -> torch.Tensor:
    """c rounded to bf16 (round to nearest even) in the forward, identity in
    the backward: the operand a bf16-MFMA layer multiplies with while its
    fp32 master parameter receives the gradient unchanged."""
    return c + (c.to(torch.bfloat16).to(c.dtype) - c).detach()


def mlp_forward(x: torch.Tensor, coeff_list, use_recurrence: bool = False,
                bf16_coeffs: bool = False, layer_fns=None) -> torch.Tensor:
    """A stack of ChebyKAN layers as in KANSequential (kan/layers/base.py:144-153).

    ``bf16_coeffs`` evaluates each layer with its coefficients rounded to
    bf16 (the bf16-compute case; the reference itself cannot run bf16
    coefficients, so its fp32 math on the rounded operands is the check).
    ``layer_fns``: per layer, a function (h, coeffs) -> output standing in
    for another layer type (a Jacobi / Hermite layer of family_oracle), or
    None for the ChebyKAN layer."""
    h = x
    for l, c in enumerate(coeff_list):
        fn = layer_fns[l] if layer_fns is not None else None
        if fn is not None:
            h = fn(h, c)
        else:
            h = layer_forward(h, round_bf16_ste(c) if bf16_coeffs else c, use_recurrence)
    return h


def train_steps(x: torch.Tensor, target: torch.Tensor, coeff_list, steps: int,
                loss: str = "mse", optimizer: str = "adam", lr: float = 0.01,
                weight_decay: float = 0.0, eps: float = 1e-8, bf16_coeffs: bool = False,
                return_state: bool = False, layer_fns=None):
    """The reference training loop (README.md:55-69) on the restatement.

    zero_grad -> forward -> loss (MSELoss / CrossEntropyLoss, mean reduction)
    -> backward -> torch.optim.Adam / SGD step, ``steps`` times.
    Returns (final coefficient list, list of per-step losses), plus the
    optimizer's per-parameter state list (exp_avg, exp_avg_sq, step for
    Adam) when ``return_state``.  ``layer_fns`` as in mlp_forward.
    """
    params = [c.detach().clone().requires_grad_(True) for c in coeff_list]
    if optimizer == "adam":
        opt = torch.optim.Adam(params, lr=lr, eps=eps, weight_decay=weight_decay)
    else:
        opt = torch.optim.SGD(params, lr=lr, weight_decay=weight_decay)
    losses = []
    for _ in range(steps):
        opt.zero_grad()
        out = mlp_forward(x, params, bf16_coeffs=bf16_coeffs, layer_fns=layer_fns)
        if loss == "mse":
            l = F.mse_loss(out, target)
        else:
            l = F.cross_entropy(out, target)
        l.backward()
        opt.step()
        losses.append(float(l.detach()))
    coeffs = [p.detach() for p in params]
    if return_state:
        return coeffs, losses, [dict(opt.state[p]) for p in params]
    return coeffs, losses


# ---------------------------------------------------------------------------
# fp64 restatement from the mathematics (numpy), used to pin the above
# ---------------------------------------------------------------------------

def cheb_T_fp64(t: np.ndarray, degree: int) -> np.ndarray:
    """T_n(t) = cos(n arccos t) in float64, shape t.shape + (degree+1,)."""
    th = np.arccos(np.clip(np.asarray(t, dtype=np.float64), -1.0, 1.0))
    n = np.arange(degree + 1, dtype=np.float64)
    return np.cos(th[..., None] * n)


def cheb_T_powersum_fp64(t: np.ndarray, degree: int) -> np.ndarray:
    """T_n(t) from the explicit sum
    T_n(t) = (n/2) sum_{k=0}^{floor(n/2)} (-1)^k (n-k-1)! / (k! (n-2k)!) (2t)^(n-2k),
    T_0 = 1.  Independent of both the recurrence and the trigonometric form.
    """
    t = np.asarray(t, dtype=np.float64)
    out = np.empty(t.shape + (degree + 1,), dtype=np.float64)
    out[..., 0] = 1.0
    for n in range(1, degree + 1):
        acc = np.zeros_like(t)
        for k in range(n // 2 + 1):
            c = (-1) ** k * math.factorial(n - k - 1) / (math.factorial(k) * math.factorial(n - 2 * k))
            acc = acc + c * (2.0 * t) ** (n - 2 * k)
        out[..., n] = 0.5 * n * acc
    return out


def cheb_U_fp64(t: np.ndarray, degree: int) -> np.ndarray:
    """U_n(t) = sin((n+1) th) / sin(th), th = arccos t, float64 (|t| < 1)."""
    th = np.arccos(np.asarray(t, dtype=np.float64))
    n = np.arange(degree + 1, dtype=np.float64)
    return np.sin((n + 1) * th[..., None]) / np.sin(th)[..., None]


def forward_fp64(x: np.ndarray, c: np.ndarray) -> np.ndarray:
    """y = sum_{i,d} T_d(tanh x) C[i,o,d] in float64 (vectorised)."""
    x = np.asarray(x, dtype=np.float64)
    c = np.asarray(c, dtype=np.float64)
    basis = cheb_T_fp64(np.tanh(x), c.shape[2] - 1)
    return np.einsum("bid,iod->bo", basis, c)


def backward_fp64(x: np.ndarray, c: np.ndarray, dy: np.ndarray):
    """Analytic gradients in float64.

    dC[i,o,d] = sum_b T_d(t[b,i]) dy[b,o]
    dx[b,i]   = (1 - t^2) sum_{o,d} dy[b,o] C[i,o,d] d U_{d-1}(t)
    """
    x = np.asarray(x, dtype=np.float64)
    c = np.asarray(c, dtype=np.float64)
    dy = np.asarray(dy, dtype=np.float64)
    deg = c.shape[2] - 1
    t = np.tanh(x)
    basis = cheb_T_fp64(t, deg)
    dc = np.einsum("bid,bo->iod", basis, dy)
    # d/dt T_d = d U_{d-1}(t), evaluated by the U recurrence (valid on [-1,1])
    u = np.zeros(t.shape + (deg + 1,))
    dT = np.zeros(t.shape + (deg + 1,))
    if deg >= 1:
        u_prev, u_cur = np.zeros_like(t), np.ones_like(t)   # U_{-1}, U_0
        for d in range(1, deg + 1):
            dT[..., d] = d * u_cur
            u_prev, u_cur = u_cur, 2 * t * u_cur - u_prev
    g = np.einsum("bo,iod->bid", dy, c)
    dx = (g * dT).sum(-1) * (1 - t * t)
    return dx, dc


def forward_bruteforce(x, c) -> np.ndarray:
    """Pure-Python triple loop (tiny shapes only): y_o = sum_i sum_d C[i,o,d] T_d(tanh x_i).

    Mirrors the layer semantics stated by the reference's symbolic export
    (kan/utils/symbolic.py:315-341), with T_d from the three-term recurrence.
    """
    x = np.asarray(x, dtype=np.float64)
    c = np.asarray(c, dtype=np.float64)
    bsz, in_dim = x.shape
    _, out_dim, dd = c.shape
    y = np.zeros((bsz, out_dim))
    for b in range(bsz):
        for o in range(out_dim):
            s = 0.0
            for i in range(in_dim):
                t = math.tanh(x[b, i])
                tm, tc = 1.0, t
                for d in range(dd):
                    td = 1.0 if d == 0 else (t if d == 1 else None)
                    if d >= 2:
                        tm, tc = tc, 2 * t * tc - tm
                        td = tc
                    s += c[i, o, d] * td
            y[b, o] = s
    return y
