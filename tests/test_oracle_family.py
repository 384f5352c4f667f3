"""Pins of the Jacobi / Hermite oracle (oracle/family_oracle.py) and of the
library's host-side change of basis (ckan_basis_to_chebyshev).  CPU only.

Each oracle function is checked against an independent source: scipy's
eval_jacobi, numpy.polynomial (legval, hermval, hermeval), special values,
brute-force sums and central finite differences.
"""
import ctypes
import math

import numpy as np
import numpy.polynomial.chebyshev as npc
import numpy.polynomial.hermite as nph
import numpy.polynomial.hermite_e as nphe
import numpy.polynomial.legendre as npl
import pytest
import scipy.special as sps
import torch

from kan_amd import _lib
from oracle import family_oracle as fo

JACOBI_PARAMS = [(0.0, 0.0), (0.5, -0.5), (1.5, 0.5), (-0.5, -0.5), (2.0, 3.0), (-0.9, 0.7)]
T = np.linspace(-1.0, 1.0, 41)


def _unit(n):
    e = np.zeros(n + 1)
    e[n] = 1.0
    return e


@pytest.mark.parametrize("alpha,beta", JACOBI_PARAMS)
def test_jacobi_basis_matches_scipy(alpha, beta):
    deg = 16
    ref = np.stack([sps.eval_jacobi(n, alpha, beta, T) for n in range(deg + 1)], -1)
    got = fo.jacobi_basis(torch.tensor(T, dtype=torch.float64).view(-1, 1), deg, alpha, beta)
    np.testing.assert_allclose(got.numpy()[:, 0, :], ref, rtol=1e-10, atol=1e-10 * np.abs(ref).max())
    np.testing.assert_allclose(fo.jacobi_fp64(T, deg, alpha, beta), ref, rtol=1e-9,
                               atol=1e-9 * np.abs(ref).max())
    # swapping the parameters is a different family unless they are equal
    if alpha != beta:
        swapped = fo.jacobi_basis(torch.tensor(T).view(-1, 1), deg, beta, alpha).numpy()[:, 0, :]
        assert np.abs(swapped - ref).max() > 1e-3


@pytest.mark.parametrize("alpha,beta", JACOBI_PARAMS)
def test_jacobi_special_value_at_one(alpha, beta):
    # P_n^(a,b)(1) = C(n + a, n)
    vals = fo.jacobi_basis(torch.ones(1, 1, dtype=torch.float64), 12, alpha, beta).numpy()[0, 0]
    for n in range(13):
        expect = math.gamma(n + alpha + 1) / (math.gamma(n + 1) * math.gamma(alpha + 1))
        assert vals[n] == pytest.approx(expect, rel=1e-12)


def test_legendre_is_jacobi_zero_zero():
    got = fo.jacobi_fp64(T, 10, 0.0, 0.0)
    for n in range(11):
        np.testing.assert_allclose(got[:, n], npl.legval(T, _unit(n)), atol=1e-12)


@pytest.mark.parametrize("scaling,ref_fn", [("physicist", nph.hermval), ("probabilist", nphe.hermeval)])
def test_hermite_basis_matches_numpy(scaling, ref_fn):
    deg = 16
    t = 3.0 * T
    ref = np.stack([ref_fn(t, _unit(n)) for n in range(deg + 1)], -1)
    got = fo.hermite_basis(torch.tensor(t).view(-1, 1), deg, scaling).numpy()[:, 0, :]
    np.testing.assert_allclose(got, ref, rtol=1e-11, atol=1e-11 * np.abs(ref).max())
    np.testing.assert_allclose(fo.hermite_fp64(t, deg, scaling), ref, rtol=1e-9,
                               atol=1e-9 * np.abs(ref).max())


def test_hermite_values_at_zero():
    h = fo.hermite_basis(torch.zeros(1, 1, dtype=torch.float64), 12, "physicist").numpy()[0, 0]
    he = fo.hermite_basis(torch.zeros(1, 1, dtype=torch.float64), 12, "probabilist").numpy()[0, 0]
    for n in range(13):
        if n % 2:
            assert h[n] == 0 and he[n] == 0
        else:
            m = n // 2
            assert h[n] == (-1) ** m * math.factorial(n) / math.factorial(m)
            assert he[n] == (-1) ** m * math.factorial(n) / (math.factorial(m) * 2 ** m)


def test_hermite_normalize_modes():
    x = torch.linspace(-4, 4, 9, dtype=torch.float64).view(-1, 1)
    assert torch.equal(fo.hermite_normalize(x), torch.tanh(x) * 3.0)
    assert torch.equal(fo.hermite_normalize(x, (-2.0, 6.0), False), torch.tanh(x) * 3.0)
    aff = fo.hermite_normalize(x, (-2.0, 6.0), True)
    torch.testing.assert_close(aff, 6.0 / 8.0 * (x + 2.0) - 3.0)


@pytest.mark.parametrize("family,alpha,beta", [("jacobi", 1.5, 0.5), ("hermite", 0, 0),
                                               ("hermite_e", 0, 0)])
def test_family_forward_matches_brute_force(family, alpha, beta):
    g = torch.Generator().manual_seed(3)
    B, I, O, deg = 3, 4, 2, 5
    x = torch.randn(B, I, generator=g, dtype=torch.float64)
    c = torch.randn(I, O, deg + 1, generator=g, dtype=torch.float64)
    y = fo.family_forward(x, c, family, alpha, beta).numpy()
    s = 1.0 if family == "jacobi" else 3.0
    for b in range(B):
        for o in range(O):
            acc = 0.0
            for i in range(I):
                t = s * math.tanh(float(x[b, i]))
                for d in range(deg + 1):
                    if family == "jacobi":
                        p = sps.eval_jacobi(d, alpha, beta, t)
                    elif family == "hermite":
                        p = nph.hermval(t, _unit(d))
                    else:
                        p = nphe.hermeval(t, _unit(d))
                    acc += float(c[i, o, d]) * p
            assert y[b, o] == pytest.approx(acc, rel=1e-10)
    np.testing.assert_allclose(fo.family_forward_fp64(x.numpy(), c.numpy(), family, alpha, beta),
                               y, rtol=1e-9)


@pytest.mark.parametrize("family,alpha,beta", [("jacobi", 0.5, -0.5), ("jacobi", 2.0, 3.0),
                                               ("hermite", 0, 0), ("hermite_e", 0, 0)])
def test_family_backward_autograd_matches_closed_form_and_fd(family, alpha, beta):
    g = torch.Generator().manual_seed(5)
    B, I, O, deg = 4, 3, 2, 7
    x = torch.randn(B, I, generator=g, dtype=torch.float64)
    c = torch.randn(I, O, deg + 1, generator=g, dtype=torch.float64)
    dy = torch.randn(B, O, generator=g, dtype=torch.float64)
    _, dx, dc = fo.family_forward_backward(x, c, dy, family, alpha, beta)
    dx64, dc64 = fo.family_backward_fp64(x.numpy(), c.numpy(), dy.numpy(), family, alpha, beta)
    np.testing.assert_allclose(dx.numpy(), dx64, rtol=1e-9, atol=1e-9 * np.abs(dx64).max())
    np.testing.assert_allclose(dc.numpy(), dc64, rtol=1e-9, atol=1e-12)
    # central differences of the fp64 forward pin the derivative identities
    h = 1e-6
    xn = x.numpy()
    for b in range(B):
        for i in range(I):
            xp, xm = xn.copy(), xn.copy()
            xp[b, i] += h
            xm[b, i] -= h
            fd = (fo.family_forward_fp64(xp, c.numpy(), family, alpha, beta)
                  - fo.family_forward_fp64(xm, c.numpy(), family, alpha, beta)) / (2 * h)
            assert float((fd[b] * dy.numpy()[b]).sum()) == pytest.approx(dx64[b, i], rel=1e-5, abs=1e-6)


@pytest.mark.parametrize("family", ["hermite", "hermite_e"])
def test_hermite_affine_domain_map_forward_backward(family):
    """A finite domain with normalize_domain maps x linearly onto [-3, 3]
    (kan/basis/hermite.py:102-112): the op-for-op forward equals the fp64 form
    on that map, and the fp64 gradients (chain factor 6 / (hi - lo)) match
    autograd and central differences, also for x outside the domain."""
    g = torch.Generator().manual_seed(6)
    B, I, O, deg, dom = 5, 3, 2, 6, (-2.0, 5.0)
    x = torch.rand(B, I, generator=g, dtype=torch.float64) * 11 - 4  # some outside [lo, hi]
    c = torch.randn(I, O, deg + 1, generator=g, dtype=torch.float64)
    dy = torch.randn(B, O, generator=g, dtype=torch.float64)
    y = fo.family_forward(x, c, family, domain=dom)
    t = 6.0 / (dom[1] - dom[0]) * (x - dom[0]) - 3.0
    assert torch.allclose(fo.hermite_normalize(x, dom), t)
    np.testing.assert_allclose(y.numpy(), fo.family_forward_fp64(x.numpy(), c.numpy(), family, domain=dom),
                               rtol=1e-10, atol=1e-10)
    # the default (tanh) map gives a different function
    assert not np.allclose(y.numpy(), fo.family_forward_fp64(x.numpy(), c.numpy(), family))
    _, dx, dc = fo.family_forward_backward(x, c, dy, family, domain=dom)
    dx64, dc64 = fo.family_backward_fp64(x.numpy(), c.numpy(), dy.numpy(), family, domain=dom)
    np.testing.assert_allclose(dx.numpy(), dx64, rtol=1e-9, atol=1e-9 * np.abs(dx64).max())
    np.testing.assert_allclose(dc.numpy(), dc64, rtol=1e-9, atol=1e-12)
    h = 1e-6
    xn = x.numpy()
    for b in range(B):
        for i in range(I):
            xp, xm = xn.copy(), xn.copy()
            xp[b, i] += h
            xm[b, i] -= h
            fd = (fo.family_forward_fp64(xp, c.numpy(), family, domain=dom)
                  - fo.family_forward_fp64(xm, c.numpy(), family, domain=dom)) / (2 * h)
            assert float((fd[b] * dy.numpy()[b]).sum()) == pytest.approx(dx64[b, i], rel=1e-5, abs=1e-6)


# ---- library host function: the change of basis used by the HIP path ------

def _M(family, deg, alpha=0.0, beta=0.0, scale=1.0):
    lib = _lib.load()
    spec = _lib.make_spec(family, deg, alpha, beta, scale)
    M = (ctypes.c_double * ((deg + 1) ** 2))()
    assert lib.ckan_basis_to_chebyshev(spec, M) == 0, lib.ckan_last_error()
    return np.array(M[:]).reshape(deg + 1, deg + 1)


@pytest.mark.parametrize("family,alpha,beta,scale", [
    (_lib.CKAN_BASIS_JACOBI, 0.0, 0.0, 1.0), (_lib.CKAN_BASIS_JACOBI, 1.5, 0.5, 1.0),
    (_lib.CKAN_BASIS_JACOBI, -0.5, -0.5, 1.0), (_lib.CKAN_BASIS_HERMITE, 0, 0, 3.0),
    (_lib.CKAN_BASIS_HERMITE_E, 0, 0, 3.0)])
@pytest.mark.parametrize("deg", [0, 1, 4, 9, 16])
def test_basis_to_chebyshev_is_exact(family, alpha, beta, scale, deg):
    M = _M(family, deg, alpha, beta, scale)
    u = np.cos(np.linspace(0.05, 3.1, 37))
    T = np.stack([npc.chebval(u, _unit(k)) for k in range(deg + 1)], -1)
    t = scale * u
    if family == _lib.CKAN_BASIS_JACOBI:
        P = np.stack([sps.eval_jacobi(n, alpha, beta, t) for n in range(deg + 1)], -1)
    elif family == _lib.CKAN_BASIS_HERMITE:
        P = np.stack([nph.hermval(t, _unit(n)) for n in range(deg + 1)], -1)
    else:
        P = np.stack([nphe.hermeval(t, _unit(n)) for n in range(deg + 1)], -1)
    np.testing.assert_allclose(T @ M.T, P, rtol=1e-10, atol=1e-10 * np.abs(P).max())
    assert np.allclose(np.triu(M, 1), 0.0)  # lower triangular


def test_basis_to_chebyshev_identity_and_validation():
    lib = _lib.load()
    assert np.array_equal(_M(_lib.CKAN_BASIS_CHEBYSHEV, 8), np.eye(9))
    M = (ctypes.c_double * 4)()
    assert lib.ckan_basis_to_chebyshev(_lib.make_spec(_lib.CKAN_BASIS_JACOBI, 1, -1.0, 0.0), M) == \
        _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_basis_to_chebyshev(_lib.make_spec(9, 1), M) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_basis_to_chebyshev(_lib.make_spec(_lib.CKAN_BASIS_HERMITE, 17), M) == \
        _lib.CKAN_ERR_UNSUPPORTED
    assert lib.ckan_basis_to_chebyshev(_lib.make_spec(_lib.CKAN_BASIS_HERMITE, 1, 0, 0, math.inf), M) \
        == _lib.CKAN_ERR_INVALID_ARG
    d = _lib.make_desc(8, 4, 3, 5, 0, 0)
    spec = _lib.make_spec(_lib.CKAN_BASIS_HERMITE, 4)  # degree mismatch: rejected before launch
    assert lib.ckan_pack_coeffs_basis(d, spec, 1, 16, None) == _lib.CKAN_ERR_INVALID_ARG
    spec = _lib.make_spec(_lib.CKAN_BASIS_HERMITE, 5)
    assert lib.ckan_coeff_grad_from_chebyshev(d, spec, 16, 16, 1, None) == _lib.CKAN_ERR_INVALID_ARG


def test_family_layers_mirror_reference_surface():
    import kan_amd
    torch.manual_seed(7)
    j = kan_amd.JacobiKANLayer(5, 3, 4, alpha=0.5, beta=1.0)
    torch.manual_seed(7)
    ref = torch.empty(5, 3, 5)
    torch.nn.init.normal_(ref, mean=0.0, std=1.0 / (5 * 5))
    assert torch.equal(j.jacobi_coeffs.detach(), ref)
    assert list(j.state_dict()) == ["jacobi_coeffs"]
    assert j.get_coefficients() is j.jacobi_coeffs
    assert j.basis.name == "Jacobi-4-0.5-1.0"
    assert repr(j) == "JacobiKANLayer(input_dim=5, output_dim=3, degree=4, alpha=0.5, beta=1.0)"
    with pytest.raises(ValueError):
        kan_amd.JacobiKANLayer(2, 2, 3, alpha=-1.0)
    h = kan_amd.get_layer("hermitekan", input_dim=2, output_dim=4, degree=3, scaling="probabilist")
    assert list(h.state_dict()) == ["hermite_coeffs"]
    assert h.basis.name == "Hermite-3-probabilist" and h.basis.domain == (-math.inf, math.inf)
    assert h.get_analytical_form()["scaling"] == "probabilist"
    with pytest.raises(ValueError):
        kan_amd.HermiteKANLayer(2, 2, 3, scaling="other")
    assert set(kan_amd.LAYER_REGISTRY) >= {"chebykan", "jacobikan", "hermitekan"}
    assert isinstance(kan_amd.get_basis("jacobi", degree=3, alpha=0.2), kan_amd.JacobiBasis)
    # the affine input map of a finite normalised domain is refused loudly
    hd = kan_amd.HermiteKANLayer(2, 2, 3, domain=(-1.0, 1.0))
    with pytest.raises(RuntimeError):
        hd(torch.zeros(1, 2))
