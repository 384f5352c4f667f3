"""Basis plug-in interface, the Chebyshev basis and the Jacobi / Hermite bases.

Mirrors the reference's ``BasisFunction`` ABC (kan/basis/base.py:7-94) and
``ChebyshevBasis`` (kan/basis/chebyshev.py:8-172): same constructor, names,
``forward(x, coefficients)`` and ``basis_functions(x)`` contracts, and the
registry name ``'chebyshev'`` (kan/basis/__init__.py:19-46).  The math runs
in the HIP library; both the closed form (default) and the recurrence
variant of the reference compute T_n(t), which this build evaluates with the
three-term recurrence in fp32 registers.

``JacobiBasis`` (kan/basis/jacobi.py:14-188) and ``HermiteBasis``
(kan/basis/hermite.py:14-233) keep their reference constructors, names and
registry names ``'jacobi'`` / ``'hermite'``.  Their ``forward`` runs the same
HIP kernels: the library re-expresses the family's coefficients in the
Chebyshev basis of the same tanh input (an exact change of basis) and maps
the coefficient gradient back.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
import math
from typing import Optional, Tuple

import torch

from . import _lib
from . import functional as F


class BasisFunction(ABC):
    """Interface of a KAN basis (kan/basis/base.py:7-94)."""

    @abstractmethod
    def __init__(self, degree: int, **kwargs):
        self.degree = degree

    @abstractmethod
    def forward(self, x: torch.Tensor, coefficients: torch.Tensor) -> torch.Tensor:
        """[B, in] x, [in, out, degree+1] coefficients -> [B, out]."""

    @abstractmethod
    def basis_functions(self, x: torch.Tensor) -> torch.Tensor:
        """[B, in] -> [B, in, degree+1]."""

    @property
    @abstractmethod
    def name(self) -> str: ...

    @property
    @abstractmethod
    def domain(self) -> Tuple[float, float]: ...

    def normalize_input(self, x: torch.Tensor) -> torch.Tensor:
        """Default squash to (-1, 1) (kan/basis/base.py:67-78)."""
        return torch.tanh(x)

    def _spec_or_none(self):
        spec = getattr(self, "spec", None)
        return spec() if callable(spec) else None

    def derivative(self, x: torch.Tensor, coefficients: torch.Tensor, order: int = 1) -> torch.Tensor:
        """[B, out]: sum over inputs of the order-th x-derivative of each
        univariate function f_{i,o}(x_i) = sum_n C[i,o,n] P_n(normalize_input(x_i))
        (kan/basis/base.py:81-94, kan/basis/chebyshev.py:174-228).

        Divergence: the reference's Chebyshev derivative coefficients are wrong
        from degree 3 on and leave out the input map's chain factor; this is the
        exact derivative in x, the same quantity KANLayer.compute_derivatives
        returns (degree + order <= 256; 16 for the Jacobi / Hermite bases and
        under a Hermite basis' finite-domain affine map)."""
        x = x.reshape(-1, coefficients.shape[0])
        aff = getattr(self, "_affine", None)
        return F.derivatives(x, coefficients, self._spec_or_none(), order,
                             getattr(self, "compute", "fp32"), aff() if callable(aff) else None)

    def numerical_derivative(self, x: torch.Tensor, coefficients: torch.Tensor, order: int = 1,
                             eps: float = 1e-6) -> torch.Tensor:
        """Central finite differences of forward in x, shifting every input by
        the same step, so order 1 approximates derivative(x, coefficients, 1)
        (kan/basis/base.py:96-125).  Divergence: for order > 1 the reference
        differentiates its first derivative as if it were coefficients; this
        applies the central difference order times to the forward."""
        if order < 0:
            raise ValueError(f"order must be >= 0, got {order}")
        with torch.no_grad():
            def diff(k: int, xs: torch.Tensor) -> torch.Tensor:
                if k == 0:
                    return self.forward(xs, coefficients)
                return (diff(k - 1, xs + eps) - diff(k - 1, xs - eps)) / (2 * eps)
            return diff(order, x)

    @staticmethod
    def to_numpy(x):
        """torch tensor -> numpy array (kan/basis/base.py:127-139)."""
        if isinstance(x, torch.Tensor):
            return x.detach().cpu().numpy()
        return x

    @staticmethod
    def normalize_domain(x: torch.Tensor, src_domain: Tuple[float, float],
                         dst_domain: Tuple[float, float]) -> torch.Tensor:
        """Linear map of src_domain onto dst_domain (kan/basis/base.py:178-196)."""
        src_min, src_max = src_domain
        dst_min, dst_max = dst_domain
        return ((x - src_min) / (src_max - src_min)) * (dst_max - dst_min) + dst_min


class ChebyshevBasis(BasisFunction):
    """Chebyshev polynomials of the first kind, T_n(tanh x).

    ``forward`` fuses tanh, the basis and the 'bid,iod->bo' contraction in
    one HIP path (kan/basis/chebyshev.py:80-101); ``compute`` selects fp32
    MFMA (default, the reference's precision) or bf16 MFMA with fp32
    accumulation.
    """

    def __init__(self, degree: int, domain: Tuple[float, float] = (-1, 1),
                 use_recurrence: bool = False, compute: str = "fp32"):
        super().__init__(degree)
        self._domain = domain
        self.use_recurrence = use_recurrence
        F.compute_code(compute)
        self.compute = compute
        self.arange = torch.arange(0, degree + 1, dtype=torch.float32)

    @property
    def name(self) -> str:
        return f"Chebyshev-{self.degree}"

    @property
    def domain(self) -> Tuple[float, float]:
        return self._domain

    def normalize_input(self, x: torch.Tensor) -> torch.Tensor:
        return torch.tanh(x)

    def forward(self, x: torch.Tensor, coefficients: torch.Tensor) -> torch.Tensor:
        x = x.view(-1, coefficients.shape[0])
        return F.chebykan(x, coefficients, self.compute)

    def basis_functions(self, x: torch.Tensor) -> torch.Tensor:
        """T_0..T_degree of an already-normalised x (kan/basis/chebyshev.py:103-117)."""
        return F.chebyshev_basis(x, self.degree)


class JacobiBasis(BasisFunction):
    """Jacobi polynomials P_n^(alpha, beta)(tanh x), alpha, beta > -1."""

    def __init__(self, degree: int, alpha: float = 0.0, beta: float = 0.0,
                 domain: Tuple[float, float] = (-1, 1), compute: str = "fp32"):
        super().__init__(degree)
        if alpha <= -1 or beta <= -1:
            raise ValueError(f"Parameters must satisfy α, β > -1, got α={alpha}, β={beta}")
        self.alpha = alpha
        self.beta = beta
        self._domain = domain
        F.compute_code(compute)
        self.compute = compute
        self.arange = torch.arange(0, degree + 1, dtype=torch.float32)

    @property
    def name(self) -> str:
        return f"Jacobi-{self.degree}-{self.alpha}-{self.beta}"

    @property
    def domain(self) -> Tuple[float, float]:
        return self._domain

    def normalize_input(self, x: torch.Tensor) -> torch.Tensor:
        return torch.tanh(x)

    def spec(self) -> _lib.CkanBasisSpec:
        return _lib.make_spec(_lib.CKAN_BASIS_JACOBI, self.degree, self.alpha, self.beta, 1.0)

    def forward(self, x: torch.Tensor, coefficients: torch.Tensor) -> torch.Tensor:
        x = x.view(-1, coefficients.shape[0])
        return F.family_kan(x, coefficients, self.spec(), self.compute)

    def basis_functions(self, x: torch.Tensor) -> torch.Tensor:
        """P_0..P_degree of an already-normalised x (kan/basis/jacobi.py:119-188)."""
        return F.family_basis(x, self.spec())


class HermiteBasis(BasisFunction):
    """Hermite polynomials, physicists' H_n or probabilists' He_n, of 3 tanh(x)."""

    def __init__(self, degree: int, scaling: str = "physicist",
                 domain: Optional[Tuple[float, float]] = None, normalize_domain: bool = True,
                 compute: str = "fp32"):
        super().__init__(degree)
        if scaling not in ["physicist", "probabilist"]:
            raise ValueError(f"Invalid scaling: {scaling}. "
                             f"Must be one of ['physicist', 'probabilist']")
        self.scaling = scaling
        self._normalize_domain = normalize_domain
        self._domain = domain or (-float("inf"), float("inf"))
        F.compute_code(compute)
        self.compute = compute
        self.arange = torch.arange(0, degree + 1, dtype=torch.float32)

    @property
    def name(self) -> str:
        return f"Hermite-{self.degree}-{self.scaling}"

    @property
    def domain(self) -> Tuple[float, float]:
        return self._domain

    def _affine_map(self) -> bool:
        """True when the reference maps a finite domain linearly onto [-3, 3]
        (kan/basis/hermite.py:102-112) instead of using 3 tanh(x)."""
        lo, hi = self._domain
        return bool(self._normalize_domain and math.isfinite(lo) and math.isfinite(hi))

    def normalize_input(self, x: torch.Tensor) -> torch.Tensor:
        if self._affine_map():
            lo, hi = self._domain
            return 6.0 / (hi - lo) * (x - lo) - 3.0
        return torch.tanh(x) * 3.0

    def spec(self) -> _lib.CkanBasisSpec:
        fam = _lib.CKAN_BASIS_HERMITE if self.scaling == "physicist" else _lib.CKAN_BASIS_HERMITE_E
        return _lib.make_spec(fam, self.degree, 0.0, 0.0, 3.0)

    def _affine(self):
        """(a, b) with u = a x + b: the finite-domain map onto [-3, 3] of
        kan/basis/hermite.py:102-112, z = 6 (x - lo) / (hi - lo) - 3, written
        as z = 3 u with u on [-1, 1] (the basis then runs at scale 3, as for
        the 3 tanh(x) map); None for the tanh map."""
        if not self._affine_map():
            return None
        lo, hi = self._domain
        return 2.0 / (hi - lo), -(hi + lo) / (hi - lo)

    def forward(self, x: torch.Tensor, coefficients: torch.Tensor) -> torch.Tensor:
        x = x.view(-1, coefficients.shape[0])
        return F.family_kan(x, coefficients, self.spec(), self.compute, self._affine())

    def basis_functions(self, x: torch.Tensor) -> torch.Tensor:
        """H_0..H_degree (or He_n) of an already-normalised x (kan/basis/hermite.py:141-233)."""
        return F.family_basis(x, self.spec())


BASIS_REGISTRY = {"chebyshev": ChebyshevBasis, "jacobi": JacobiBasis, "hermite": HermiteBasis}


def get_basis(name: str, **kwargs) -> BasisFunction:
    """Name lookup as in kan/basis/__init__.py:31-46 (ValueError if unknown)."""
    if name not in BASIS_REGISTRY:
        raise ValueError(f"Unknown basis function: {name}. Available: {', '.join(BASIS_REGISTRY)}")
    return BASIS_REGISTRY[name](**kwargs)
