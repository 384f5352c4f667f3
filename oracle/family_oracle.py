"""CPU oracle for the Jacobi and Hermite KAN layers.

TEST INFRASTRUCTURE ONLY.  This module checks the HIP path of
``kan_amd.JacobiKANLayer`` / ``HermiteKANLayer``; nothing in the product
imports it.

* op-for-op torch (CPU) restatements of the reference, in its op order:
    - ``jacobi_basis``        follows kan/basis/jacobi.py:147-188
    - ``hermite_basis``       follows kan/basis/hermite.py:158-193 ('physicist')
                              and :195-233 ('probabilist')
    - ``hermite_normalize``   follows kan/basis/hermite.py:85-116
    - ``family_forward``      follows kan/basis/jacobi.py:96-117 and
                              kan/basis/hermite.py:118-139 (tanh / 3 tanh,
                              basis, einsum('bid,iod->bo'))
    - ``family_forward_backward`` is torch autograd through that restatement
* fp64 restatements from the mathematics, used to pin the above:
    - ``jacobi_fp64``   the explicit binomial sum of P_n^(alpha, beta)
    - ``hermite_fp64``  the explicit sums of H_n and He_n
    - ``family_backward_fp64``  the closed-form input derivative through
      P_n' (Jacobi: (n + a + b + 1)/2 P_{n-1}^(a+1, b+1); Hermite: 2n H_{n-1},
      n He_{n-1}) and tanh.

Parity status: every function is pinned in tests/test_oracle_family.py
against scipy.special.eval_jacobi, numpy.polynomial (hermval, hermeval,
legval), special values, brute-force sums and finite differences.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch

__all__ = [
    "jacobi_basis", "hermite_basis", "hermite_normalize", "family_basis", "family_forward",
    "family_forward_backward", "jacobi_fp64", "hermite_fp64", "family_forward_fp64",
    "family_backward_fp64",
]


# ---------------------------------------------------------------------------
# op-for-op torch restatement (CPU)
# ---------------------------------------------------------------------------

def jacobi_basis(x: torch.Tensor, degree: int, alpha: float, beta: float) -> torch.Tensor:
    """[B, in] -> [B, in, degree+1] (kan/basis/jacobi.py:159-188)."""
    b, i = x.shape
    cols = [torch.ones(b, i, dtype=x.dtype)]
    if degree > 0:
        cols.append(((alpha + beta + 2) * x + (alpha - beta)) / 2)
        for n in range(2, degree + 1):
            nf = float(n)
            ab_sum = alpha + beta
            ab_diff = alpha ** 2 - beta ** 2
            common_term = 2 * nf + ab_sum - 1
            term1 = (2 * nf + ab_sum) * (2 * nf + ab_sum - 2) * x + ab_diff
            coef1 = common_term * term1
            coef2 = -2 * (nf + alpha - 1) * (nf + beta - 1) * (2 * nf + ab_sum)
            denom = 2 * nf * (nf + ab_sum) * (2 * nf + ab_sum - 2)
            cols.append((coef1 * cols[n - 1] + coef2 * cols[n - 2]) / denom)
    return torch.stack(cols, dim=2)


def hermite_basis(x: torch.Tensor, degree: int, scaling: str = "physicist") -> torch.Tensor:
    """[B, in] -> [B, in, degree+1] (kan/basis/hermite.py:171-193, 209-233)."""
    cols = [torch.ones_like(x)]
    if degree > 0:
        cols.append(2 * x if scaling == "physicist" else x.clone())
        for n in range(2, degree + 1):
            if scaling == "physicist":
                cols.append(2 * x * cols[n - 1] - 2 * (n - 1) * cols[n - 2])
            else:
                cols.append(x * cols[n - 1] - (n - 1) * cols[n - 2])
    return torch.stack(cols, dim=2)


def hermite_normalize(x: torch.Tensor, domain: Optional[Tuple[float, float]] = None,
                      normalize_domain: bool = True) -> torch.Tensor:
    """kan/basis/hermite.py:101-116."""
    lo, hi = domain or (-float("inf"), float("inf"))
    if normalize_domain and (lo, hi) != (-float("inf"), float("inf")):
        if np.isfinite(lo) and np.isfinite(hi):
            return 6.0 / (hi - lo) * (x - lo) - 3.0
    return torch.tanh(x) * 3.0


def family_basis(t: torch.Tensor, family: str, degree: int, alpha: float = 0.0,
                 beta: float = 0.0) -> torch.Tensor:
    if family == "jacobi":
        return jacobi_basis(t, degree, alpha, beta)
    return hermite_basis(t, degree, "physicist" if family == "hermite" else "probabilist")


def family_forward(x: torch.Tensor, coeffs: torch.Tensor, family: str, alpha: float = 0.0,
                   beta: float = 0.0, domain: Optional[Tuple[float, float]] = None,
                   normalize_domain: bool = True) -> torch.Tensor:
    """y = einsum('bid,iod->bo', P(map(x)), C); map = tanh (Jacobi) or the
    Hermite input map of hermite_normalize (3 tanh, or the affine map of a
    finite domain) (jacobi.py:96-117, hermite.py:118-139)."""
    x = x.view(-1, coeffs.shape[0])
    t = torch.tanh(x) if family == "jacobi" else hermite_normalize(x, domain, normalize_domain)
    basis = family_basis(t, family, coeffs.shape[2] - 1, alpha, beta)
    return torch.einsum("bid,iod->bo", basis, coeffs)


def family_forward_backward(x: torch.Tensor, coeffs: torch.Tensor, dy: torch.Tensor, family: str,
                            alpha: float = 0.0, beta: float = 0.0,
                            domain: Optional[Tuple[float, float]] = None,
                            normalize_domain: bool = True):
    xr = x.detach().clone().requires_grad_(True)
    cr = coeffs.detach().clone().requires_grad_(True)
    y = family_forward(xr, cr, family, alpha, beta, domain, normalize_domain)
    y.backward(dy)
    return y.detach(), xr.grad.detach(), cr.grad.detach()


# ---------------------------------------------------------------------------
# fp64 restatement from the mathematics
# ---------------------------------------------------------------------------

def _gbinom(a: float, k: int) -> float:
    """Generalised binomial coefficient C(a, k) for real a, integer k >= 0."""
    r = 1.0
    for j in range(k):
        r *= (a - j) / (j + 1)
    return r


def jacobi_fp64(t: np.ndarray, degree: int, alpha: float, beta: float) -> np.ndarray:
    """P_n^(a,b)(t) = sum_s C(n+a, n-s) C(n+b, s) ((t-1)/2)^s ((t+1)/2)^(n-s)."""
    t = np.asarray(t, dtype=np.float64)
    out = np.empty(t.shape + (degree + 1,))
    for n in range(degree + 1):
        acc = np.zeros_like(t)
        for s in range(n + 1):
            acc += (_gbinom(n + alpha, n - s) * _gbinom(n + beta, s)
                    * ((t - 1) / 2) ** s * ((t + 1) / 2) ** (n - s))
        out[..., n] = acc
    return out


def hermite_fp64(t: np.ndarray, degree: int, scaling: str = "physicist") -> np.ndarray:
    """H_n(t) = n! sum_m (-1)^m (2t)^(n-2m) / (m! (n-2m)!);
    He_n(t) = n! sum_m (-1)^m t^(n-2m) / (m! (n-2m)! 2^m)."""
    t = np.asarray(t, dtype=np.float64)
    out = np.empty(t.shape + (degree + 1,))
    for n in range(degree + 1):
        acc = np.zeros_like(t)
        for m in range(n // 2 + 1):
            if scaling == "physicist":
                term = (-1) ** m * (2 * t) ** (n - 2 * m) / (math.factorial(m) * math.factorial(n - 2 * m))
            else:
                term = ((-1) ** m * t ** (n - 2 * m)
                        / (math.factorial(m) * math.factorial(n - 2 * m) * 2 ** m))
            acc += term
        out[..., n] = math.factorial(n) * acc
    return out


def _family_fp64(t, family, degree, alpha, beta):
    if family == "jacobi":
        return jacobi_fp64(t, degree, alpha, beta)
    return hermite_fp64(t, degree, "physicist" if family == "hermite" else "probabilist")


def _family_deriv_fp64(t, family, degree, alpha, beta):
    """d/dt P_n(t) for n = 0..degree, from the derivative identities."""
    out = np.zeros(np.shape(t) + (degree + 1,))
    if degree == 0:
        return out
    if family == "jacobi":
        lower = jacobi_fp64(t, degree - 1, alpha + 1, beta + 1)
        for n in range(1, degree + 1):
            out[..., n] = (n + alpha + beta + 1) / 2 * lower[..., n - 1]
    else:
        phys = family == "hermite"
        lower = hermite_fp64(t, degree - 1, "physicist" if phys else "probabilist")
        for n in range(1, degree + 1):
            out[..., n] = (2 * n if phys else n) * lower[..., n - 1]
    return out


def _input_map_fp64(x: np.ndarray, family: str, domain):
    """(t, dt/dx) of the layer's input map in float64: tanh (Jacobi), 3 tanh
    (Hermite), or for Hermite with a finite domain (lo, hi) the affine map
    t = 6 (x - lo) / (hi - lo) - 3."""
    x = np.asarray(x, dtype=np.float64)
    if family != "jacobi" and domain is not None:
        lo, hi = domain
        a = 6.0 / (hi - lo)
        return a * (x - lo) - 3.0, np.full_like(x, a)
    s = 1.0 if family == "jacobi" else 3.0
    u = np.tanh(x)
    return s * u, s * (1.0 - u * u)


def family_forward_fp64(x: np.ndarray, c: np.ndarray, family: str, alpha: float = 0.0,
                        beta: float = 0.0, domain=None) -> np.ndarray:
    t, _ = _input_map_fp64(x, family, domain)
    return np.einsum("bid,iod->bo", _family_fp64(t, family, c.shape[2] - 1, alpha, beta), c)


def family_backward_fp64(x: np.ndarray, c: np.ndarray, dy: np.ndarray, family: str,
                         alpha: float = 0.0, beta: float = 0.0, domain=None):
    """(dx, dC) of family_forward_fp64 for upstream gradient dy."""
    t, dtdx = _input_map_fp64(x, family, domain)
    deg = c.shape[2] - 1
    basis = _family_fp64(t, family, deg, alpha, beta)
    dbasis = _family_deriv_fp64(t, family, deg, alpha, beta)
    g = np.einsum("bo,iod->bid", dy, c)
    dx = np.einsum("bid,bid->bi", g, dbasis) * dtdx
    dc = np.einsum("bid,bo->iod", basis, dy)
    return dx, dc
