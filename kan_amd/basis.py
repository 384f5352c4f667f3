"""Basis plug-in interface and the Chebyshev basis.

Mirrors the reference's ``BasisFunction`` ABC (kan/basis/base.py:7-94) and
``ChebyshevBasis`` (kan/basis/chebyshev.py:8-172): same constructor, names,
``forward(x, coefficients)`` and ``basis_functions(x)`` contracts, and the
registry name ``'chebyshev'`` (kan/basis/__init__.py:19-46).  The math runs
in the HIP library; both the closed form (default) and the recurrence
variant of the reference compute T_n(t), which this build evaluates with the
three-term recurrence in fp32 registers.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Tuple

import torch

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


BASIS_REGISTRY = {"chebyshev": ChebyshevBasis}


def get_basis(name: str, **kwargs) -> BasisFunction:
    """Name lookup as in kan/basis/__init__.py:31-46 (ValueError if unknown)."""
    if name not in BASIS_REGISTRY:
        raise ValueError(f"Unknown basis function: {name}. Available: {', '.join(BASIS_REGISTRY)}")
    return BASIS_REGISTRY[name](**kwargs)
