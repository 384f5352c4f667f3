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
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Any, Dict, List, Optional

import torch
import torch.nn as nn

from .basis import BasisFunction, ChebyshevBasis


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


class KANSequential(nn.Sequential):
    """Sequential container of KAN layers (kan/layers/base.py:144-166)."""

    def get_analytical_form(self) -> List[Dict[str, Any]]:
        return [m.get_analytical_form() for m in self if isinstance(m, KANLayer)]


LAYER_REGISTRY = {"chebykan": ChebyKANLayer}


def get_layer(name: str, **kwargs) -> KANLayer:
    """Name lookup as in kan/layers/__init__.py:30-45 (ValueError if unknown)."""
    if name not in LAYER_REGISTRY:
        raise ValueError(f"Unknown layer: {name}. Available: {', '.join(LAYER_REGISTRY)}")
    return LAYER_REGISTRY[name](**kwargs)
