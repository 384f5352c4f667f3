"""kan_amd: the ChebyKAN layer hot path of 0xEodum/KAN, MI355X (gfx950) native.

Public surface (mirrors the reference's names for this path):
    ChebyKANLayer, JacobiKANLayer, HermiteKANLayer, KANLayer, KANSequential,
    get_layer, LAYER_REGISTRY
    ChebyshevBasis, JacobiBasis, HermiteBasis, BasisFunction, get_basis, BASIS_REGISTRY
    optim.SGD, optim.Adam (fused HIP steps)
    ResidentExecutor (whole training steps of a layer stack, resident on one GPU)
    functional.chebykan (autograd op)

All compute runs in the in-tree HIP library ``libckan_gfx950.so`` (C-ABI in
include/chebykan.h); there is no CPU fallback.
"""
from .basis import (BASIS_REGISTRY, BasisFunction, ChebyshevBasis, HermiteBasis, JacobiBasis,
                    get_basis)
from .layers import (LAYER_REGISTRY, ChebyKANLayer, HermiteKANLayer, JacobiKANLayer, KANLayer,
                     KANSequential, get_layer)
from . import functional, optim
from .executor import ResidentExecutor

__version__ = "0.1.0"

__all__ = [
    "ChebyKANLayer", "JacobiKANLayer", "HermiteKANLayer", "KANLayer", "KANSequential",
    "get_layer", "LAYER_REGISTRY",
    "ChebyshevBasis", "JacobiBasis", "HermiteBasis", "BasisFunction", "get_basis",
    "BASIS_REGISTRY",
    "functional", "optim", "ResidentExecutor", "__version__",
]
