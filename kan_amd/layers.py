"""Drop-in ChebyKAN layer and its container.

``ChebyKANLayer`` keeps the reference constructor
``(input_dim, output_dim, degree, use_recurrence=False, init_scale=None)``
(kan/layers/chebykan.py:21-22), the single parameter ``cheby_coeffs``
[in, out, degree+1] fp32 initialised ``normal_(0, std=init_scale or
1/(in*(degree+1)))`` in the same RNG order (chebykan.py:46-51), so a seeded
construction yields bit-identical coefficients and ``state_dict`` keys.
``forward`` does ``x.view(-1, in)`` (chebykan.py:64) and runs the HIP path.
The extra keyword ``compute`` ('fp32' default, or 'bf16') selects the MFMA
precision.

``JacobiKANLayer`` (kan/layers/jacobikan.py:10-120) and ``HermiteKANLayer``
(kan/layers/hermitekan.py:10-125) mirror their reference constructors and
parameters (``jacobi_coeffs`` / ``hermite_coeffs``, same init order) and run
on the same kernels through the change of basis in ``kan_amd.basis``.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any, Dict, List, Optional, Tuple

import torch
import torch.nn as nn

from . import functional as F
from .basis import BasisFunction, ChebyshevBasis, HermiteBasis, JacobiBasis


class KANLayer(nn.Module, ABC):
    """Base class of KAN layers (kan/layers/base.py:11-100)."""

    @abstractmethod
    def __init__(self, input_dim: int, output_dim: int, basis_function: BasisFunction, **kwargs):
        super().__init__()
        self.input_dim = input_dim
        self.output_dim = output_dim
        self.basis_function = basis_function

    @abstractmethod
    def forward(self, x: torch.Tensor) -> torch.Tensor: ...

    @property
    def basis(self) -> BasisFunction:
        return self.basis_function

    @abstractmethod
    def get_analytical_form(self) -> Dict[str, Any]: ...

    @abstractmethod
    def get_coefficients(self) -> torch.Tensor: ...

    def _basis_spec(self):
        spec = getattr(self.basis_function, "spec", None)
        return spec() if callable(spec) else None

    def _compute_mode(self) -> str:
        return getattr(self.basis_function, "compute", "fp32")

    def _input_affine(self):
        """(a, b) of the basis' affine input map u = a x + b, or None for tanh."""
        aff = getattr(self.basis_function, "_affine", None)
        return aff() if callable(aff) else None

    def compute_derivatives(self, x: torch.Tensor, order: int = 1) -> torch.Tensor:
        """[batch, output_dim]: sum over inputs i of the order-th derivative in
        x_i of each univariate function f_{i,o} (kan/layers/base.py:102-114).

        Divergence: the reference evaluates ChebyshevBasis.derivative, whose
        coefficients are wrong from degree 3 on and which differentiates in
        tanh(x) without the chain factor; this returns the exact x-derivative
        (a Chebyshev series of degree degree + order: degree + order <= 256,
        or 16 for the Jacobi / Hermite layers; a Hermite layer with a finite
        domain differentiates through its affine map, chain factor included)."""
        x = x.reshape(-1, self.input_dim)
        return F.derivatives(x, self.get_coefficients(), self._basis_spec(), order,
                             self._compute_mode(), self._input_affine())

    def jacobian(self, x: torch.Tensor) -> torch.Tensor:
        """[batch, output_dim, input_dim]: d y[b, o] / d x[b, i] (kan/layers/base.py:116-141).

        Divergence: the reference fills column i with compute_derivatives of x
        with the other inputs zeroed, which adds their derivatives at 0 (and
        the reference's derivative is itself inexact); this is the exact
        Jacobian.  Computed in fp32; not differentiable."""
        x = x.reshape(-1, self.input_dim)
        return F.jacobian(x, self.get_coefficients(), self._basis_spec(), self._input_affine())


class ChebyKANLayer(KANLayer):
    """KAN layer with a tanh-squashed Chebyshev basis (kan/layers/chebykan.py:10-101)."""

    def __init__(self, input_dim: int, output_dim: int, degree: int,
                 use_recurrence: bool = False, init_scale: Optional[float] = None,
                 compute: str = "fp32"):
        basis_function = ChebyshevBasis(degree=degree, use_recurrence=use_recurrence,
                                        compute=compute)
        super().__init__(input_dim=input_dim, output_dim=output_dim,
                         basis_function=basis_function)
        self.degree = degree
        init_scale = init_scale or 1.0 / (input_dim * (degree + 1))
        self.cheby_coeffs = nn.Parameter(torch.empty(input_dim, output_dim, degree + 1))
        nn.init.normal_(self.cheby_coeffs, mean=0.0, std=init_scale)

    @property
    def compute(self) -> str:
        return self.basis_function.compute

    @compute.setter
    def compute(self, value: str) -> None:
        from .functional import compute_code
        compute_code(value)
        self.basis_function.compute = value

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.view(-1, self.input_dim)
        return self.basis_function.forward(x, self.cheby_coeffs)

    def get_analytical_form(self) -> Dict[str, Any]:
        return {
            "type": "ChebyKANLayer",
            "input_dim": self.input_dim,
            "output_dim": self.output_dim,
            "degree": self.degree,
            "basis": self.basis_function.name,
            "coefficients": self.cheby_coeffs.detach().cpu().numpy(),
        }

    def get_coefficients(self) -> torch.Tensor:
        return self.cheby_coeffs

    def extra_repr(self) -> str:
        return f"input_dim={self.input_dim}, output_dim={self.output_dim}, degree={self.degree}"


class _ComputeMixin:
    @property
    def compute(self) -> str:
        return self.basis_function.compute

    @compute.setter
    def compute(self, value: str) -> None:
        from .functional import compute_code
        compute_code(value)
        self.basis_function.compute = value


class JacobiKANLayer(_ComputeMixin, KANLayer):
    """KAN layer with a tanh-squashed Jacobi basis (kan/layers/jacobikan.py:10-120)."""

    def __init__(self, input_dim: int, output_dim: int, degree: int, alpha: float = 0.0,
                 beta: float = 0.0, init_scale: Optional[float] = None, compute: str = "fp32"):
        if alpha <= -1 or beta <= -1:
            raise ValueError(f"Parameters must satisfy α, β > -1, got α={alpha}, β={beta}")
        basis_function = JacobiBasis(degree=degree, alpha=alpha, beta=beta, compute=compute)
        super().__init__(input_dim=input_dim, output_dim=output_dim,
                         basis_function=basis_function)
        self.degree = degree
        self.alpha = alpha
        self.beta = beta
        init_scale = init_scale or 1.0 / (input_dim * (degree + 1))
        self.jacobi_coeffs = nn.Parameter(torch.empty(input_dim, output_dim, degree + 1))
        nn.init.normal_(self.jacobi_coeffs, mean=0.0, std=init_scale)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.view(-1, self.input_dim)
        return self.basis_function.forward(x, self.jacobi_coeffs)

    def get_analytical_form(self) -> Dict[str, Any]:
        return {
            "type": "JacobiKANLayer",
            "input_dim": self.input_dim,
            "output_dim": self.output_dim,
            "degree": self.degree,
            "alpha": self.alpha,
            "beta": self.beta,
            "basis": self.basis_function.name,
            "coefficients": self.jacobi_coeffs.detach().cpu().numpy(),
        }

    def get_coefficients(self) -> torch.Tensor:
        return self.jacobi_coeffs

    def extra_repr(self) -> str:
        return (f"input_dim={self.input_dim}, output_dim={self.output_dim}, degree={self.degree}, "
                f"alpha={self.alpha}, beta={self.beta}")


class HermiteKANLayer(_ComputeMixin, KANLayer):
    """KAN layer with a Hermite basis of 3 tanh(x) (kan/layers/hermitekan.py:10-125)."""

    def __init__(self, input_dim: int, output_dim: int, degree: int, scaling: str = "physicist",
                 domain: Optional[Tuple[float, float]] = None, normalize_domain: bool = True,
                 init_scale: Optional[float] = None, compute: str = "fp32"):
        basis_function = HermiteBasis(degree=degree, scaling=scaling, domain=domain,
                                      normalize_domain=normalize_domain, compute=compute)
        super().__init__(input_dim=input_dim, output_dim=output_dim,
                         basis_function=basis_function)
        self.degree = degree
        self.scaling = scaling
        self.domain = domain
        self.normalize_domain = normalize_domain
        init_scale = init_scale or 1.0 / (input_dim * (degree + 1))
        self.hermite_coeffs = nn.Parameter(torch.empty(input_dim, output_dim, degree + 1))
        nn.init.normal_(self.hermite_coeffs, mean=0.0, std=init_scale)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x.view(-1, self.input_dim)
        return self.basis_function.forward(x, self.hermite_coeffs)

    def get_analytical_form(self) -> Dict[str, Any]:
        return {
            "type": "HermiteKANLayer",
            "input_dim": self.input_dim,
            "output_dim": self.output_dim,
            "degree": self.degree,
            "scaling": self.scaling,
            "domain": self.domain,
            "normalize_domain": self.normalize_domain,
            "basis": self.basis_function.name,
            "coefficients": self.hermite_coeffs.detach().cpu().numpy(),
        }

    def get_coefficients(self) -> torch.Tensor:
        return self.hermite_coeffs

    def extra_repr(self) -> str:
        domain_str = f", domain={self.domain}" if self.domain else ""
        normalize_str = f", normalize_domain={self.normalize_domain}"
        return (f"input_dim={self.input_dim}, output_dim={self.output_dim}, "
                f"degree={self.degree}, scaling={self.scaling}{domain_str}{normalize_str}")


class KANSequential(nn.Sequential):
    """Sequential container of KAN layers (kan/layers/base.py:144-193)."""

    def get_analytical_form(self) -> List[Dict[str, Any]]:
        return [m.get_analytical_form() for m in self if isinstance(m, KANLayer)]

    def visualize_network(self, **kwargs):
        """Not provided, as in the reference (kan/layers/base.py:168-179)."""
        raise NotImplementedError("Network visualization is not implemented yet")

    def jacobian(self, x: torch.Tensor) -> torch.Tensor:
        """Not provided, as in the reference (kan/layers/base.py:181-193)."""
        raise NotImplementedError("Network Jacobian computation is not implemented yet")


LAYER_REGISTRY = {"chebykan": ChebyKANLayer, "jacobikan": JacobiKANLayer,
                  "hermitekan": HermiteKANLayer}


def get_layer(name: str, **kwargs) -> KANLayer:
    """Name lookup as in kan/layers/__init__.py:30-45 (ValueError if unknown)."""
    if name not in LAYER_REGISTRY:
        raise ValueError(f"Unknown layer: {name}. Available: {', '.join(LAYER_REGISTRY)}")
    return LAYER_REGISTRY[name](**kwargs)
