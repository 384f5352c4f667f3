"""GPU parity of KANLayer.compute_derivatives / jacobian (HIP path through the
C-ABI: ckan_derivative_coeffs + the ChebyKAN forward, ckan_jacobian) against
the CPU oracle oracle/derivative_oracle.py (fp64 autograd through the
reference's forward).

Tolerances (norm-wise, ||a - b|| / ||b||):
  fp32 path:  1e-5 for the derivatives, the Jacobian and their gradients
  bf16 MFMA path:  2e-2 (the derivative layer's forward in bf16)

Divergence from the reference (documented in kan_amd/layers.py): these are
the exact x-derivatives; the reference's are not (see the oracle's header).
"""
import numpy as np
import pytest
import torch

import kan_amd
from kan_amd import _lib
from oracle import derivative_oracle as do
from oracle import family_oracle as fo

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    n = b.norm().item()
    return (a - b).norm().item() / (n if n > 0 else 1.0)


def _inputs(seed, B, I, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(B, I, generator=g) * scale


CHEB_CASES = [
    # B, I, O, deg, order
    (64, 16, 12, 4, 1),
    (300, 40, 24, 8, 1),
    (300, 40, 24, 8, 2),
    (128, 32, 20, 5, 3),
    (1024, 64, 48, 8, 1),    # pipelined forward of the derivative layer (degree 9 -> P = 16)
    (700, 48, 40, 12, 4),    # degree 16 derivative layer
]


@pytest.mark.parametrize("B,I,O,deg,order", CHEB_CASES)
def test_chebykan_derivatives_fp32(B, I, O, deg, order):
    torch.manual_seed(B + deg + order)
    layer = kan_amd.ChebyKANLayer(I, O, deg).cuda()
    x = _inputs(order, B, I)
    got = layer.compute_derivatives(x.cuda(), order=order)
    ref = do.derivatives(x, layer.cheby_coeffs.detach().cpu(), order)
    assert got.shape == (B, O)
    assert _rel(got, ref) <= FP32_TOL


@pytest.mark.parametrize("order", [1, 2])
def test_chebykan_derivatives_bf16(order):
    B, I, O, deg = 2048, 128, 96, 8
    torch.manual_seed(7)
    layer = kan_amd.ChebyKANLayer(I, O, deg, compute="bf16").cuda()
    x = _inputs(3, B, I)
    got = layer.compute_derivatives(x.cuda(), order=order)
    ref = do.derivatives(x, layer.cheby_coeffs.detach().cpu(), order)
    assert _rel(got, ref) <= BF16_TOL


def test_order_zero_is_the_forward():
    torch.manual_seed(3)
    layer = kan_amd.ChebyKANLayer(20, 10, 6).cuda()
    x = _inputs(1, 50, 20).cuda()
    torch.testing.assert_close(layer.compute_derivatives(x, order=0), layer(x))


@pytest.mark.parametrize("B,I,O,deg", [(37, 9, 7, 5), (256, 64, 32, 8), (5, 3, 130, 15)])
def test_chebykan_jacobian(B, I, O, deg):
    torch.manual_seed(B)
    layer = kan_amd.ChebyKANLayer(I, O, deg).cuda()
    x = _inputs(2, B, I)
    J = layer.jacobian(x.cuda())
    ref = do.jacobian(x, layer.cheby_coeffs.detach().cpu())
    assert J.shape == (B, O, I)
    assert _rel(J, ref) <= FP32_TOL
    # its sum over inputs is compute_derivatives(order=1)
    assert _rel(J.sum(dim=2), layer.compute_derivatives(x.cuda(), 1)) <= FP32_TOL


FAMILY_CASES = [
    ("jacobi", dict(alpha=0.5, beta=-0.25), 1),
    ("jacobi", dict(alpha=0.0, beta=0.0), 2),
    ("hermite", dict(scaling="physicist"), 1),
    ("hermite_e", dict(scaling="probabilist"), 2),
]


@pytest.mark.parametrize("family,kw,order", FAMILY_CASES)
def test_family_derivatives_and_jacobian(family, kw, order):
    B, I, O, deg = 300, 24, 20, 6
    torch.manual_seed(11 + order)
    if family == "jacobi":
        layer = kan_amd.JacobiKANLayer(I, O, deg, **kw).cuda()
        fwd = lambda xx, cc: fo.family_forward(xx, cc, "jacobi", kw["alpha"], kw["beta"])
    else:
        layer = kan_amd.HermiteKANLayer(I, O, deg, **kw).cuda()
        fwd = lambda xx, cc: fo.family_forward(xx, cc, family)
    c = layer.get_coefficients().detach().cpu()
    x = _inputs(4, B, I, scale=0.8)
    got = layer.compute_derivatives(x.cuda(), order=order)
    assert _rel(got, do.derivatives(x, c, order, fwd)) <= FP32_TOL
    assert _rel(layer.jacobian(x.cuda()), do.jacobian(x, c, fwd)) <= FP32_TOL


AFFINE_CASES = [
    ("hermite", dict(scaling="physicist", domain=(-1.5, 2.5)), 1),
    ("hermite", dict(scaling="physicist", domain=(-1.5, 2.5)), 3),
    ("hermite_e", dict(scaling="probabilist", domain=(-3.0, 1.0)), 2),
]


@pytest.mark.parametrize("family,kw,order", AFFINE_CASES)
def test_hermite_finite_domain_derivatives_and_jacobian(family, kw, order):
    """A Hermite layer with a finite domain maps x by z = 6 (x - lo) / (hi -
    lo) - 3 (kan/basis/hermite.py:102-112): its x-derivatives carry the
    constant chain factor (6 / (hi - lo))^order and lower the degree, against
    fp64 autograd through the oracle's forward with that map, and the
    derivative of H_n(z) = 2n H_{n-1}(z) (He_n: n He_{n-1}) at order 1."""
    B, I, O, deg = 300, 24, 20, 6
    print(f"hermite affine derivatives {family} {kw} order={order}", flush=True)
    torch.manual_seed(21 + order)
    layer = kan_amd.HermiteKANLayer(I, O, deg, **kw).cuda()
    fwd = lambda xx, cc: fo.family_forward(xx, cc, family, domain=kw["domain"])
    c = layer.get_coefficients().detach().cpu()
    lo, hi = kw["domain"]
    x = lo + (hi - lo) * torch.rand(B, I, generator=torch.Generator().manual_seed(5 + order))
    got = layer.compute_derivatives(x.cuda(), order=order)
    assert _rel(got, do.derivatives(x, c, order, fwd)) <= FP32_TOL
    J = layer.jacobian(x.cuda())
    assert _rel(J, do.jacobian(x, c, fwd)) <= FP32_TOL
    if order == 1:  # the closed form: dx of the fp64 backward with dy = e_o, summed over i
        dx, _ = fo.family_backward_fp64(x.numpy(), c.double().numpy(), np.ones((B, O)), family,
                                        domain=kw["domain"])
        assert _rel(got.sum(dim=1), torch.from_numpy(dx.sum(axis=1))) <= FP32_TOL
    # outside the operator's reach: degree + order above 16
    with pytest.raises(_lib.CkanError) as e:
        kan_amd.HermiteKANLayer(8, 4, 15, domain=(-1.0, 1.0)).cuda().compute_derivatives(
            x[:, :8].cuda(), order=2)
    assert e.value.code == _lib.CKAN_ERR_UNSUPPORTED


def test_derivatives_are_differentiable():
    """d/dC and d/dx of a loss of compute_derivatives (the physics-informed use)."""
    B, I, O, deg = 200, 16, 12, 6
    torch.manual_seed(5)
    layer = kan_amd.ChebyKANLayer(I, O, deg).cuda()
    x = _inputs(6, B, I)
    w = torch.randn(B, O)
    xd = x.cuda().requires_grad_(True)
    (layer.compute_derivatives(xd, order=2) * w.cuda()).sum().backward()
    xr = x.double().requires_grad_(True)
    cr = layer.cheby_coeffs.detach().cpu().double().requires_grad_(True)
    yr = do.chebykan_forward64(xr, cr)
    d2 = torch.stack([torch.autograd.grad(
        torch.autograd.grad(yr[:, o].sum(), xr, create_graph=True)[0].sum(), xr,
        create_graph=True)[0].sum(1) for o in range(O)], 1)
    (d2 * w.double()).sum().backward()
    assert _rel(layer.cheby_coeffs.grad, cr.grad) <= FP32_TOL
    assert _rel(xd.grad, xr.grad) <= FP32_TOL


def _derivatives_graph(x, c, order):
    """sum_i d^order y[b, o] / d x[b, i]^order in fp64 with c kept in the graph
    (each y[b, o] is a sum of univariate functions, so the repeated gradient
    of the column sum is the per-input derivative)."""
    xr = x.double().requires_grad_(True)
    y = do.chebykan_forward64(xr, c)
    cols = []
    for o in range(y.shape[1]):
        g = y[:, o].sum()
        for _ in range(order):
            d = torch.autograd.grad(g, xr, create_graph=True)[0]
            g = d.sum()
        cols.append(d.sum(1))
    return torch.stack(cols, 1)


@pytest.mark.parametrize("B,I,O,deg,order", [
    (64, 8, 6, 14, 3),      # degree 17 derivative layer: the row-by-row operator
    (100, 12, 10, 20, 1),   # degree 20 layer (vector-ALU forward)
    (50, 6, 5, 40, 2),
])
def test_long_derivative_series_fp32(B, I, O, deg, order):
    """Past degree + order 16 the derivative coefficients come from the
    row-by-row device operator and the derivative layer runs the vector-ALU
    forward: values, coefficient and input gradients, and the Jacobian."""
    print(f"long derivative series B={B} I={I} O={O} deg={deg} order={order}", flush=True)
    torch.manual_seed(B + deg)
    layer = kan_amd.ChebyKANLayer(I, O, deg).cuda()
    x = _inputs(deg, B, I)
    got = layer.compute_derivatives(x.cuda(), order=order)
    c64 = layer.cheby_coeffs.detach().cpu().double()
    ref = do.derivatives(x, c64, order)
    assert _rel(got, ref) <= FP32_TOL
    # coefficient gradient of sum(w * derivative): the adjoint operator
    w = torch.randn(B, O, generator=torch.Generator().manual_seed(1))
    layer.cheby_coeffs.grad = None
    (layer.compute_derivatives(x.cuda(), order=order) * w.cuda()).sum().backward()
    cr = c64.clone().requires_grad_(True)
    (_derivatives_graph(x, cr, order) * w.double()).sum().backward()
    assert _rel(layer.cheby_coeffs.grad, cr.grad) <= FP32_TOL
    if order == 1 or deg + 1 > 16:
        jac = layer.jacobian(x.cuda())
        xr = x.double().requires_grad_(True)
        yr = do.chebykan_forward64(xr, c64)
        jr = torch.stack([torch.autograd.grad(yr[:, o].sum(), xr, retain_graph=True)[0]
                          for o in range(O)], 1)
        assert _rel(jac, jr) <= FP32_TOL


def test_derivative_errors():
    x = torch.randn(10, 8, device="cuda")
    with pytest.raises(ValueError):
        kan_amd.ChebyKANLayer(8, 4, 14).cuda().compute_derivatives(x, order=-1)
    with pytest.raises(_lib.CkanError) as e:  # degree + order above 256
        kan_amd.ChebyKANLayer(8, 4, 250).cuda().compute_derivatives(x, order=7)
    assert e.value.code == _lib.CKAN_ERR_UNSUPPORTED
    with pytest.raises(_lib.CkanError) as e:  # family bases stop at degree + order 16
        kan_amd.JacobiKANLayer(8, 4, 15).cuda().compute_derivatives(x, order=2)
    assert e.value.code == _lib.CKAN_ERR_UNSUPPORTED
    layer64 = kan_amd.ChebyKANLayer(8, 4, 3).cuda().double()
    with pytest.raises(RuntimeError):
        layer64.compute_derivatives(x.double(), order=1)


def test_basis_derivative_and_numerical_derivative():
    """ChebyshevBasis.derivative is the exact x-derivative summed over inputs
    (what compute_derivatives returns); numerical_derivative (central
    differences of forward, every input shifted together) approximates it, at
    order 1 and, unlike the reference's recursion, at order 2."""
    import kan_amd
    torch.manual_seed(3)
    m = kan_amd.ChebyKANLayer(6, 4, 5).cuda()
    b = m.basis
    x = (torch.rand(32, 6) * 2 - 1).cuda()
    c = m.cheby_coeffs.detach()
    for order in (1, 2):
        exact = b.derivative(x, c, order)
        assert torch.allclose(exact, m.compute_derivatives(x, order))
        c64 = c.double().cpu()
        # fp64 finite differences of the oracle's forward, for the same quantity
        from oracle import chebykan_oracle as orc
        h = 1e-4
        f = lambda xs: torch.from_numpy(orc.forward_fp64(xs.numpy(), c64.numpy()))
        xc = x.double().cpu()
        ref = ((f(xc + h) - f(xc - h)) / (2 * h) if order == 1
               else (f(xc + h) - 2 * f(xc) + f(xc - h)) / (h * h))
        assert ((exact.double().cpu() - ref).norm() / ref.norm()).item() <= 1e-4
        num = b.numerical_derivative(x, c, order, eps=1e-2)
        assert ((num.double().cpu() - ref).norm() / ref.norm()).item() <= 5e-2
