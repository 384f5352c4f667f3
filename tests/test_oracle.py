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


def _mlp_grads_fp64(x, coeffs, target, loss):
    """fp64 loss and coefficient gradients of a ChebyKAN stack, chained by hand
    through backward_fp64 (independent of torch autograd)."""
    hs = [np.asarray(x, dtype=np.float64)]
    for c in coeffs:
        hs.append(orc.forward_fp64(hs[-1], c.numpy()))
    y = hs[-1]
    B, O = y.shape
    if loss == "mse":
        t = target.double().numpy()
        lval = ((y - t) ** 2).mean()
        dy = 2.0 * (y - t) / (B * O)
    else:
        lab = target.numpy()
        z = y - y.max(1, keepdims=True)
        p = np.exp(z) / np.exp(z).sum(1, keepdims=True)
        lval = -np.log(p[np.arange(B), lab]).mean()
        dy = p.copy()
        dy[np.arange(B), lab] -= 1.0
        dy /= B
    grads = [None] * len(coeffs)
    for l in range(len(coeffs) - 1, -1, -1):
        dh, grads[l] = orc.backward_fp64(hs[l], coeffs[l].numpy(), dy)
        dy = dh
    return lval, grads


@pytest.mark.parametrize("loss", ["mse", "ce"])
@pytest.mark.parametrize("wd", [0.0, 0.3])
def test_train_steps_one_sgd_step_closed_form(loss, wd):
    """One step of the loop is C1 = C0 - lr (dC + wd C0), with dC the fp64
    analytic gradient of the mean-reduced loss.  A missing zero_grad, a sum
    instead of a mean, or a dropped layer gradient fails this."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(24, 6, generator=g)
    coeffs = [torch.randn(6, 5, 4, generator=g) * 0.2, torch.randn(5, 3, 6, generator=g) * 0.2]
    target = torch.randn(24, 3, generator=g) if loss == "mse" else torch.randint(0, 3, (24,), generator=g)
    lr = 0.05
    lval, grads = _mlp_grads_fp64(x, coeffs, target, loss)
    c1, losses = orc.train_steps(x, target, coeffs, steps=1, loss=loss, optimizer="sgd", lr=lr,
                                 weight_decay=wd)
    assert abs(losses[0] - lval) <= 1e-5 * abs(lval)
    for l in range(2):
        want = coeffs[l].double().numpy() - lr * (grads[l] + wd * coeffs[l].double().numpy())
        delta = c1[l].double().numpy() - coeffs[l].double().numpy()
        dwant = want - coeffs[l].double().numpy()
        assert np.linalg.norm(delta - dwant) <= 1e-5 * np.linalg.norm(dwant)
    # two steps: the second gradient is taken at C1 (not accumulated onto the first)
    c2, _ = orc.train_steps(x, target, coeffs, steps=2, loss=loss, optimizer="sgd", lr=lr,
                            weight_decay=wd)
    _, grads1 = _mlp_grads_fp64(x, c1, target, loss)
    for l in range(2):
        dwant = -lr * (grads1[l] + wd * c1[l].double().numpy())
        delta = c2[l].double().numpy() - c1[l].double().numpy()
        assert np.linalg.norm(delta - dwant) <= 1e-4 * np.linalg.norm(dwant)


def test_train_steps_one_adam_step_closed_form():
    """Adam's first step: m = (1-b1) g, v = (1-b2) g^2, so
    C1 = C0 - lr g / (|g| + eps) elementwise; the returned state holds m, v."""
    g = torch.Generator().manual_seed(12)
    x = torch.randn(32, 5, generator=g)
    coeffs = [torch.randn(5, 4, 9, generator=g) * 0.1]
    target = torch.randn(32, 4, generator=g)
    lr, eps = 0.01, 1e-3
    _, grads = _mlp_grads_fp64(x, coeffs, target, "mse")
    c1, _, state = orc.train_steps(x, target, coeffs, steps=1, loss="mse", optimizer="adam", lr=lr,
                                   eps=eps, return_state=True)
    gr = grads[0]
    want = coeffs[0].double().numpy() - lr * gr / (np.abs(gr) + eps)
    assert np.abs(c1[0].double().numpy() - want).max() <= 1e-6
    assert np.allclose(state[0]["exp_avg"].double().numpy(), 0.1 * gr, rtol=1e-4, atol=1e-9)
    assert np.allclose(state[0]["exp_avg_sq"].double().numpy(), 0.001 * gr * gr, rtol=1e-3,
                       atol=1e-14)
    assert float(state[0]["step"]) == 1.0


def test_train_steps_bf16_coeffs_rounds_the_operand_only():
    """bf16_coeffs: the forward uses bf16(C) (round to nearest even), and the
    fp32 master receives the gradient taken at bf16(C) unchanged."""
    g = torch.Generator().manual_seed(13)
    x = torch.randn(16, 4, generator=g)
    c = [torch.randn(4, 3, 6, generator=g) * 0.3 + 1e-3]
    target = torch.randn(16, 3, generator=g)
    cr = [c[0].to(torch.bfloat16).float()]
    assert not torch.equal(cr[0], c[0])
    y = orc.mlp_forward(x, c, bf16_coeffs=True)
    assert np.allclose(y.double().numpy(), orc.forward_fp64(x.numpy(), cr[0].numpy()), rtol=1e-5,
                       atol=1e-6)
    lr = 0.1
    _, grads = _mlp_grads_fp64(x, cr, target, "mse")
    c1, _ = orc.train_steps(x, target, c, steps=1, loss="mse", optimizer="sgd", lr=lr,
                            bf16_coeffs=True)
    delta = c1[0].double().numpy() - c[0].double().numpy()
    assert np.linalg.norm(delta + lr * grads[0]) <= 1e-5 * np.linalg.norm(lr * grads[0])
