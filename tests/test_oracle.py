"""Pins the CPU oracle (oracle/chebykan_oracle.py) against the mathematics.

The reference ships no tests or golden vectors, so each oracle function is
checked here against something that a plausible mistake (a dropped term, a
wrong sign or index, a transposed operand) would break: special values,
T_n(cos th) = cos(n th), the explicit power-sum form of T_n, brute-force loops,
central finite differences, and torch.optim itself for the optimizer steps.
"""
import math

import numpy as np
import pytest
import torch

from oracle import chebykan_oracle as orc


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)


@pytest.mark.parametrize("deg", [0, 1, 2, 4, 8, 16])
def test_special_values(deg):
    t = torch.tensor([[1.0, -1.0, 0.0]])
    tf = orc.cheb_T_fp64(t.numpy(), deg)
    n = np.arange(deg + 1)
    assert np.allclose(tf[0, 0], 1.0)
    assert np.allclose(tf[0, 1], (-1.0) ** n)
    assert np.allclose(tf[0, 2], np.cos(n * np.pi / 2), atol=1e-12)
    tr = orc.basis_recurrence(t.double(), deg).numpy()
    assert np.array_equal(tr[0, 0], np.ones(deg + 1))
    assert np.array_equal(tr[0, 1], (-1.0) ** n)
    assert np.array_equal(tr[0, 2], np.round(np.cos(n * np.pi / 2)))


@pytest.mark.parametrize("deg", [1, 3, 4, 8, 9, 16])
def test_three_forms_of_T_agree(deg):
    rng = np.random.default_rng(deg)
    th = rng.uniform(0, np.pi, size=(7, 5))
    t = np.cos(th)
    closed = orc.cheb_T_fp64(t, deg)
    power = orc.cheb_T_powersum_fp64(t, deg)
    # T_n(cos th) = cos(n th)
    assert np.allclose(closed, np.cos(th[..., None] * np.arange(deg + 1)), atol=1e-12)
    assert np.allclose(power, closed, atol=1e-9)
    rec = orc.basis_recurrence(torch.from_numpy(t), deg).numpy()
    assert np.allclose(rec, closed, atol=1e-12)
    # the fp32 closed form (reference default) agrees to fp32 accuracy
    cf = orc.basis_closed_form(torch.from_numpy(t).float(), deg).numpy()
    assert np.max(np.abs(cf - closed)) < 5e-6 * max(1, deg)


def test_powersum_known_coefficients():
    # T_4 = 8t^4 - 8t^2 + 1, T_5 = 16t^5 - 20t^3 + 5t (textbook)
    t = np.linspace(-1, 1, 11)
    p = orc.cheb_T_powersum_fp64(t, 5)
    assert np.allclose(p[:, 4], 8 * t ** 4 - 8 * t ** 2 + 1)
    assert np.allclose(p[:, 5], 16 * t ** 5 - 20 * t ** 3 + 5 * t)


def test_U_matches_derivative_of_T():
    # d/dt T_n = n U_{n-1}
    t = np.linspace(-0.95, 0.95, 41)
    h = 1e-6
    T_p = orc.cheb_T_fp64(t + h, 8)
    T_m = orc.cheb_T_fp64(t - h, 8)
    dT = (T_p - T_m) / (2 * h)
    U = orc.cheb_U_fp64(t, 8)
    for n in range(1, 9):
        assert np.allclose(dT[:, n], n * U[:, n - 1], atol=1e-6)


def test_forward_bruteforce_and_fp64():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 4, generator=g)
    c = torch.randn(4, 5, 4, generator=g)
    y = orc.layer_forward(x, c).numpy()
    yb = orc.forward_bruteforce(x.numpy(), c.numpy())
    yf = orc.forward_fp64(x.numpy(), c.numpy())
    assert np.allclose(yb, yf, atol=1e-12)
    assert _rel(y, yb) < 1e-6
    # operand roles are not symmetric: a transposed C would not match
    c2 = c.permute(1, 0, 2).contiguous()
    assert c2.shape != c.shape or _rel(orc.layer_forward(x, c2).numpy(), yb) > 1e-2


def test_recurrence_variant_matches_closed_form():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(16, 8, generator=g)
    c = torch.randn(8, 6, 9, generator=g)
    y0 = orc.layer_forward(x, c, use_recurrence=False)
    y1 = orc.layer_forward(x, c, use_recurrence=True)
    assert _rel(y1.numpy(), y0.numpy()) < 1e-6


def test_backward_fp64_vs_finite_differences():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(3, 4))
    c = rng.normal(size=(4, 2, 6))
    dy = rng.normal(size=(3, 2))
    dx, dc = orc.backward_fp64(x, c, dy)
    h = 1e-6
    fd_x = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp = x.copy(); xp[idx] += h
        xm = x.copy(); xm[idx] -= h
        fd_x[idx] = ((orc.forward_fp64(xp, c) - orc.forward_fp64(xm, c)) * dy).sum() / (2 * h)
    assert np.allclose(dx, fd_x, rtol=1e-6, atol=1e-7)
    fd_c = np.zeros_like(c)
    for idx in np.ndindex(c.shape):
        cp = c.copy(); cp[idx] += h
        cm = c.copy(); cm[idx] -= h
        fd_c[idx] = ((orc.forward_fp64(x, cp) - orc.forward_fp64(x, cm)) * dy).sum() / (2 * h)
    assert np.allclose(dc, fd_c, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("deg", [1, 4, 8, 16])
def test_autograd_restatement_matches_analytic(deg):
    g = torch.Generator().manual_seed(deg)
    x = torch.randn(32, 12, generator=g)
    c = torch.randn(12, 7, deg + 1, generator=g) / (12 * (deg + 1))
    dy = torch.randn(32, 7, generator=g)
    y, dx, dc = orc.layer_forward_backward(x, c, dy)
    dx64, dc64 = orc.backward_fp64(x.numpy(), c.numpy(), dy.numpy())
    assert _rel(y.numpy(), orc.forward_fp64(x.numpy(), c.numpy())) < 1e-5
    assert _rel(dc.numpy(), dc64) < 1e-5
    assert _rel(dx.numpy(), dx64) < 1e-4  # closed-form acos backward is ill-conditioned near |t|=1


def test_saturation_nan_in_reference_backward():
    # Beyond |x| ~ 9.0108 fp32 tanh is exactly +-1 and the reference's
    # closed-form backward gives NaN; the analytic derivative stays finite.
    x = torch.tensor([[0.0], [3.0], [9.5], [-12.0]])
    c = torch.ones(1, 1, 9)
    dy = torch.ones(4, 1)
    _, dx, _ = orc.layer_forward_backward(x, c, dy)
    dx = dx.numpy().ravel()
    assert abs(dx[0] - (-4.0)) < 1e-5
    assert abs(dx[1] - 1.8765) < 1e-3
    assert np.isnan(dx[2]) and np.isnan(dx[3])
    dx64, _ = orc.backward_fp64(x.numpy(), c.numpy(), dy.numpy())
    assert np.all(np.isfinite(dx64))
    assert abs(float(torch.tanh(torch.tensor(orc.SATURATION_X + 1e-3)))) == 1.0


def test_init_coeffs_reproduces_parameter_init():
    torch.manual_seed(123)
    p = torch.nn.Parameter(torch.empty(5, 3, 9))
    torch.nn.init.normal_(p, mean=0.0, std=1.0 / (5 * 9))
    c = orc.init_coeffs(5, 3, 8, seed=123)
    assert torch.equal(p.detach(), c)
    # init_scale=0.0 falls back to the default because of ``or``
    c0 = orc.init_coeffs(5, 3, 8, init_scale=0.0, seed=123)
    assert torch.equal(c0, c)
    big = orc.init_coeffs(64, 64, 8, seed=7)
    assert abs(big.std().item() - 1.0 / (64 * 9)) < 0.05 / (64 * 9)


@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_adam_step_matches_torch_optim(wd):
    g = torch.Generator().manual_seed(5)
    p0 = torch.randn(40, generator=g)
    p_ref = p0.clone().requires_grad_(True)
    opt = torch.optim.Adam([p_ref], lr=0.01, weight_decay=wd)
    p = p0.clone()
    m = torch.zeros_like(p)
    v = torch.zeros_like(p)
    for step in range(1, 6):
        grad = torch.randn(40, generator=g)
        p_ref.grad = grad.clone()
        opt.step()
        orc.adam_step(p, grad, m, v, step, lr=0.01, weight_decay=wd)
        assert torch.allclose(p, p_ref.detach(), rtol=0, atol=1e-7)


def test_sgd_step_matches_torch_optim():
    g = torch.Generator().manual_seed(6)
    p0 = torch.randn(33, generator=g)
    p_ref = p0.clone().requires_grad_(True)
    opt = torch.optim.SGD([p_ref], lr=0.05)
    p = p0.clone()
    for _ in range(3):
        grad = torch.randn(33, generator=g)
        p_ref.grad = grad.clone()
        opt.step()
        orc.sgd_step(p, grad, 0.05)
    assert torch.equal(p, p_ref.detach())


def test_train_steps_cfg1_decreases_loss():
    # config 1 (README.md:42-73), shortened: the loss must fall
    torch.manual_seed(0)
    x = torch.linspace(-1, 1, 100).reshape(-1, 1)
    y = torch.sin(2 * math.pi * x)
    c = orc.init_coeffs(1, 1, 8, seed=0)
    _, losses = orc.train_steps(x, y, [c], steps=200, loss="mse", optimizer="adam", lr=0.01)
    assert losses[-1] < 0.25 * losses[0]
