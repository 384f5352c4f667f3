"""Pins of the derivative oracle (oracle/derivative_oracle.py) and of the
library's host-side derivative operator (ckan_derivative_matrix).  CPU only.

The oracle (fp64 autograd through the reference's closed-form forward) is
checked against central finite differences; the library's matrix R, built
by a different method (the operator p -> (1 - t^2) p' applied in the T basis),
is checked against the oracle and against numpy's chebder.
"""
import math

import numpy as np
import numpy.polynomial.chebyshev as npc
import pytest
import torch

from kan_amd import _lib
from oracle import derivative_oracle as do
from oracle import family_oracle as fo

FAMILIES = [
    ("chebyshev", None),
    ("jacobi", (_lib.CKAN_BASIS_JACOBI, 0.5, -0.25, 1.0)),
    ("hermite", (_lib.CKAN_BASIS_HERMITE, 0.0, 0.0, 3.0)),
    ("hermite_e", (_lib.CKAN_BASIS_HERMITE_E, 0.0, 0.0, 3.0)),
]


def _forward(family, alpha=0.0, beta=0.0):
    if family == "chebyshev":
        return do.chebykan_forward64
    return lambda x, c: fo.family_forward(x, c, family, alpha, beta)


def _spec(entry, degree):
    if entry is None:
        return None
    fam, a, b, s = entry
    return _lib.make_spec(fam, degree, a, b, s)


def _case(seed, B=7, I=3, O=4, deg=5, scale=1.5):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, I, generator=g, dtype=torch.float64) * scale
    c = torch.randn(I, O, deg + 1, generator=g, dtype=torch.float64) / (deg + 1)
    return x, c


@pytest.mark.parametrize("family,entry", FAMILIES)
@pytest.mark.parametrize("order", [1, 2])
def test_oracle_derivatives_match_finite_differences(family, entry, order):
    x, c = _case(1 + order)
    a, b = (entry[1], entry[2]) if entry else (0.0, 0.0)
    fwd = _forward(family, a, b)
    got = do.derivatives(x, c, order, fwd)
    fd = do.finite_difference(x, c, order, h=1e-3 if order == 1 else 2e-3, forward=fwd)
    scale = fd.abs().max().item()
    assert (got - fd).abs().max().item() <= 1e-5 * max(scale, 1.0)


def test_oracle_jacobian_matches_finite_differences():
    x, c = _case(5)
    J = do.jacobian(x, c)
    h = 1e-4
    for i in range(x.shape[1]):
        e = torch.zeros_like(x)
        e[:, i] = h
        fd = (do.chebykan_forward64(x + e, c) - do.chebykan_forward64(x - e, c)) / (2 * h)
        np.testing.assert_allclose(J[:, :, i].numpy(), fd.numpy(), rtol=1e-6, atol=1e-8)
    # the Jacobian's sum over inputs is compute_derivatives(order=1)
    np.testing.assert_allclose(J.sum(dim=2).numpy(), do.derivatives(x, c, 1).numpy(), atol=1e-12)


@pytest.mark.parametrize("family,entry", FAMILIES)
@pytest.mark.parametrize("order", [1, 2, 3])
def test_derivative_matrix_reproduces_oracle(family, entry, order):
    deg = 5
    x, c = _case(10 + order, deg=deg, scale=1.2)
    R = _lib.derivative_matrix(_spec(entry, deg), deg, order)
    assert R.shape == (deg + 1, deg + 1 + order)
    ck = torch.from_numpy(np.einsum("ion,nk->iok", c.numpy(), R))
    got = do.chebykan_forward64(x, ck)  # a Chebyshev layer of degree deg + order
    a, b = (entry[1], entry[2]) if entry else (0.0, 0.0)
    ref = do.derivatives(x, c, order, _forward(family, a, b))
    np.testing.assert_allclose(got.numpy(), ref.numpy(), rtol=1e-9,
                               atol=1e-9 * ref.abs().max().item())


def test_derivative_matrix_rows_follow_chebder():
    # row n of R (Chebyshev, order 1) is (1 - t^2) T_n'(t); order 2 applies it twice
    deg = 9
    t = np.linspace(-1, 1, 33)
    R1 = _lib.derivative_matrix(None, deg, 1)
    R2 = _lib.derivative_matrix(None, deg, 2)
    for n in range(deg + 1):
        e = np.zeros(deg + 1)
        e[n] = 1.0
        d1 = (1 - t * t) * npc.chebval(t, npc.chebder(e))
        np.testing.assert_allclose(npc.chebval(t, R1[n]), d1, atol=1e-12 * max(1, n * n))
        # second application: (1 - t^2) d/dt of the first
        q1 = R1[n]
        d2 = (1 - t * t) * npc.chebval(t, npc.chebder(q1))
        np.testing.assert_allclose(npc.chebval(t, R2[n]), d2, atol=1e-11 * max(1, n ** 4))
    # closed form: (1 - t^2) T_n' = n (T_{n-1} - T_{n+1}) / 2
    for n in range(1, deg + 1):
        expect = np.zeros(deg + 2)
        expect[n - 1] += n / 2
        expect[n + 1] -= n / 2
        np.testing.assert_allclose(R1[n], expect, atol=1e-14)
    np.testing.assert_array_equal(R1[0], np.zeros(deg + 2))


@pytest.mark.parametrize("deg,order", [(12, 5), (30, 2), (64, 3)])
def test_derivative_matrix_long_series_follow_chebder(deg, order):
    """Past degree + order 16 (the operator the GPU row kernels apply): row n
    of R is (1 - t^2) d/dt applied `order` times to T_n, checked through
    numpy's chebder / chebmulx in fp64, relative to each row's size."""
    R = _lib.derivative_matrix(None, deg, order)
    assert R.shape == (deg + 1, deg + 1 + order)
    for n in range(deg + 1):
        q = np.zeros(n + 1)
        q[n] = 1.0
        for _ in range(order):
            d = npc.chebder(q) if len(q) > 1 else np.zeros(1)
            q = npc.chebsub(d, npc.chebmulx(npc.chebmulx(d)))
        expect = np.zeros(deg + 1 + order)
        expect[:len(q)] = q[:deg + 1 + order]
        np.testing.assert_allclose(R[n], expect, rtol=0, atol=1e-12 * max(1.0, np.abs(expect).max()))


def test_derivative_matrix_order_zero_and_limits():
    deg = 4
    np.testing.assert_array_equal(_lib.derivative_matrix(None, deg, 0), np.eye(deg + 1))
    M = np.zeros((deg + 1) * (deg + 1))
    spec = _lib.make_spec(_lib.CKAN_BASIS_HERMITE, deg, 0.0, 0.0, 3.0)
    _lib.check(_lib.load().ckan_basis_to_chebyshev(spec, M.ctypes.data_as(
        __import__("ctypes").POINTER(__import__("ctypes").c_double))))
    np.testing.assert_allclose(_lib.derivative_matrix(spec, deg, 0), M.reshape(deg + 1, deg + 1))
    with pytest.raises(_lib.CkanError) as e:
        _lib.derivative_matrix(None, 250, 7)  # degree + order above 256
    assert e.value.code == _lib.CKAN_ERR_UNSUPPORTED
    with pytest.raises(_lib.CkanError) as e:  # family bases stop at degree + order 16
        _lib.derivative_matrix(_lib.make_spec(_lib.CKAN_BASIS_JACOBI, 12, 0.0, 0.0, 1.0), 12, 5)
    assert e.value.code == _lib.CKAN_ERR_UNSUPPORTED
    with pytest.raises(_lib.CkanError) as e:
        _lib.derivative_matrix(None, 4, -1)
    assert e.value.code == _lib.CKAN_ERR_INVALID_ARG
    with pytest.raises(_lib.CkanError):
        _lib.derivative_matrix(_lib.make_spec(_lib.CKAN_BASIS_JACOBI, 5, 0.0, 0.0, 1.0), 4, 1)


def test_reference_derivative_coefficients_diverge():
    """Documents the divergence: the reference's derivative coefficients
    (kan/basis/chebyshev.py:230-267) give T_3' = 6 T_2 - 3 T_0 and drop the
    tanh chain factor; the true d/dt T_3 is 6 T_2 + 3 T_0."""
    e = np.zeros(4)
    e[3] = 1.0
    assert npc.chebder(e).tolist() == [3.0, 0.0, 6.0]
    # the chain factor: d/dx T_1(tanh x) = 1 - tanh^2 x, R's row 1 (not 2 T_0 as the
    # reference's coefficient for n = 1, 2 n c_n, evaluated as a plain series would give)
    R = _lib.derivative_matrix(None, 3, 1)
    x = 0.7
    assert npc.chebval(math.tanh(x), R[1]) == pytest.approx(1 - math.tanh(x) ** 2, rel=1e-14)
