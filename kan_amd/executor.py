"""Resident multi-layer executor over the C-ABI (ckan_exec_*).

Trains a KANSequential of ChebyKAN, Jacobi and Hermite layers
(kan/layers/base.py:144-166) in place on one GPU: the library owns fp32 master coefficients, packed operands,
activations, tanh caches, gradients and optimizer state, and one ``step`` runs
forward, the loss and its gradient, backward and the optimizer for every
layer -- one iteration of the reference training loop (README.md:61-69).
"""
from __future__ import annotations

import ctypes
import weakref
from typing import Optional, Sequence

import torch

from . import _lib
from .functional import compute_code
from .layers import ChebyKANLayer, HermiteKANLayer, JacobiKANLayer, KANSequential

_LOSS = {"mse": _lib.CKAN_LOSS_MSE, "ce": _lib.CKAN_LOSS_CE, "cross_entropy": _lib.CKAN_LOSS_CE}
_OPT = {"sgd": _lib.CKAN_OPT_SGD, "adam": _lib.CKAN_OPT_ADAM}


_LAYER_TYPES = (ChebyKANLayer, JacobiKANLayer, HermiteKANLayer)


def check_sequential(model: KANSequential) -> list:
    """The KAN layers of ``model`` in order; ValueError when a module is not a
    ChebyKANLayer, JacobiKANLayer or HermiteKANLayer (an activation, a spline
    layer) or when the widths do not chain (layer l's input_dim != layer
    l-1's output_dim)."""
    layers = list(model)
    if not layers:
        raise ValueError("the model has no layers")
    for l, m in enumerate(layers):
        if type(m) not in _LAYER_TYPES:
            raise ValueError(f"module {l} ({type(m).__name__}) is not a ChebyKAN, Jacobi or "
                             "Hermite layer: the resident executor runs stacks of those only")
        if l and m.input_dim != layers[l - 1].output_dim:
            raise ValueError(f"layer {l} takes {m.input_dim} inputs but layer {l - 1} "
                             f"produces {layers[l - 1].output_dim}")
    return layers


def check_rows(t: torch.Tensor, rows: int, cols: int, name: str) -> None:
    """The executor reads exactly rows x cols elements of ``t``."""
    if tuple(t.shape) != (rows, cols):
        raise RuntimeError(f"{name} must be [{rows}, {cols}], got {list(t.shape)}")


def check_labels(labels: torch.Tensor, n_classes: int) -> None:
    """Class indices for the cross-entropy loss.

    torch.nn.CrossEntropyLoss raises on a label outside [0, C) and leaves rows
    labelled with its ignore_index (-100 by default) out of the loss and its
    mean.  The executor's loss kernels average over every row, so both cases
    are rejected here, before any launch, instead of training on a wrong
    loss.  Reads the labels' range (one device synchronisation when they live
    on the GPU)."""
    if labels.dtype.is_floating_point or labels.dtype == torch.bool:
        raise ValueError(f"labels must be an integer tensor, got {labels.dtype}")
    if labels.numel() == 0:
        return
    lo, hi = int(labels.min()), int(labels.max())
    if lo == -100:
        raise ValueError("labels hold -100 (CrossEntropyLoss's ignore_index): the executor's "
                         "cross-entropy has no ignored rows; drop those rows from the batch")
    if lo < 0 or hi >= n_classes:
        raise ValueError(f"labels must lie in [0, {n_classes}), found values in [{lo}, {hi}]")


def layer_basis(m):
    """(basis spec or None, affine (scale, shift) or None) of a KAN layer: the
    spec of a Jacobi / Hermite layer's basis, and the finite-domain map of a
    Hermite layer that has one (None: the tanh map)."""
    if type(m) is ChebyKANLayer:
        return None, None
    b = m.basis_function
    affine = b._affine() if hasattr(b, "_affine") else None
    return b.spec(), affine


class ResidentExecutor:
    """A resident KAN stack: ``widths`` has n_layers + 1 entries.

    ``bases``: per layer, a basis spec (``_lib.make_spec``; None for a
    ChebyKAN layer), or None for an all-ChebyKAN stack.  ``affine``: per
    layer, (scale, shift) of the input map t = scale * x + shift, or None for
    tanh (the Hermite layer's finite domain).  ``pack_each_step``: re-pack the
    coefficients at every step even where the step's dC launch keeps the
    packed operands current (two-layer cross-entropy stacks of small layers);
    the same results, for checking that path."""

    def __init__(self, widths: Sequence[int], degrees: Sequence[int], batch: int,
                 compute: str = "bf16", loss: str = "mse", optimizer: str = "sgd",
                 lr: float = 0.01, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 0.0, use_graph: bool = False, fused_small: bool = True,
                 device="cuda", bases: Optional[Sequence] = None,
                 affine: Optional[Sequence] = None, pack_each_step: bool = False):
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("ResidentExecutor runs only on a ROCm device")
        if len(widths) != len(degrees) + 1:
            raise ValueError("widths must have one more entry than degrees")
        if loss not in _LOSS:
            raise ValueError(f"loss must be one of {sorted(_LOSS)}")
        if optimizer not in _OPT:
            raise ValueError(f"optimizer must be one of {sorted(_OPT)}")
        self.widths = [int(w) for w in widths]
        self.degrees = [int(d) for d in degrees]
        self.batch = int(batch)
        self.loss_name = loss
        self.optimizer = optimizer
        self._lib = _lib.load()
        self._w = (ctypes.c_int32 * len(self.widths))(*self.widths)
        self._d = (ctypes.c_int32 * len(self.degrees))(*self.degrees)
        cfg = _lib.CkanExecConfig(
            len(self.degrees), self._w, self._d, self.batch, compute_code(compute),
            _LOSS[loss], _OPT[optimizer], 1 if use_graph else 0, float(lr), float(betas[0]),
            float(betas[1]), float(eps), float(weight_decay),
            (0 if fused_small else _lib.CKAN_EXEC_NO_FUSED_SMALL)
            | (_lib.CKAN_EXEC_PACK_EACH_STEP if pack_each_step else 0))
        n = len(self.degrees)
        specs = aff = None
        if bases is not None:
            if len(bases) != n:
                raise ValueError("bases must have one entry per layer")
            specs = (_lib.CkanBasisSpec * n)(*[
                b if b is not None else _lib.make_spec(_lib.CKAN_BASIS_CHEBYSHEV, d)
                for b, d in zip(bases, self.degrees)])
        if affine is not None:
            if len(affine) != n:
                raise ValueError("affine must have one entry per layer")
            flat = []
            for a in affine:
                flat += [0.0, 0.0] if a is None else [float(a[0]), float(a[1])]
            aff = (ctypes.c_float * (2 * n))(*flat)
        self._specs, self._aff = specs, aff
        handle = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(self._lib.ckan_exec_create_basis(ctypes.byref(cfg), specs, aff,
                                                        ctypes.byref(handle), self._stream()))
        self._h = handle
        self._loss = torch.empty((), dtype=torch.float32, device=self.device)
        self._labels_checked = None  # (weakref to the last labels checked, their _version)

    def _stream(self) -> int:
        return _lib.stream_ptr(self.device)

    def _shape(self, layer: int):
        return (self.widths[layer], self.widths[layer + 1], self.degrees[layer] + 1)

    @classmethod
    def from_sequential(cls, model: KANSequential, batch: int, **kw) -> "ResidentExecutor":
        """An executor over ``model``'s layers with their current coefficients.

        The executor's kernels run KAN layers back to back, each layer's
        output feeding the next (kan/layers/base.py:144-166), so every module
        of ``model`` must be a ChebyKANLayer, JacobiKANLayer or
        HermiteKANLayer and each layer's input_dim must equal the previous
        layer's output_dim; anything else raises ValueError before any device
        work."""
        layers = check_sequential(model)
        widths = [layers[0].input_dim] + [m.output_dim for m in layers]
        per = [layer_basis(m) for m in layers]
        if any(b is not None or a is not None for b, a in per):
            kw.setdefault("bases", [b for b, _ in per])
            kw.setdefault("affine", [a for _, a in per])
        ex = cls(widths, [m.degree for m in layers], batch, **kw)
        for l, m in enumerate(layers):
            ex.set_coeffs(l, m.get_coefficients().detach())
        return ex

    def set_coeffs(self, layer: int, coeffs: torch.Tensor) -> None:
        c = coeffs.detach().to(self.device, torch.float32).contiguous()
        if tuple(c.shape) != self._shape(layer):
            raise RuntimeError(f"layer {layer} coefficients must be {self._shape(layer)}")
        _lib.check(self._lib.ckan_exec_set_coeffs(self._h, layer, c.data_ptr(), self._stream()))
        torch.cuda.current_stream(self.device).synchronize()

    def get_coeffs(self, layer: int) -> torch.Tensor:
        out = torch.empty(self._shape(layer), dtype=torch.float32, device=self.device)
        _lib.check(self._lib.ckan_exec_get_coeffs(self._h, layer, out.data_ptr(), self._stream()))
        return out

    def step(self, x: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        """One training step; returns the step's loss as a new device scalar."""
        x, target = self._inputs(x, target)
        _lib.check(self._lib.ckan_exec_step(self._h, x.data_ptr(), target.data_ptr(),
                                            self._loss.data_ptr(), self._stream()))
        # the library writes every step's loss into the same 4 bytes: hand the
        # caller its own copy, as a torch loss tensor would be
        return self._loss.clone()

    def _x(self, x: torch.Tensor) -> torch.Tensor:
        check_rows(x, self.batch, self.widths[0], "x")
        return x.to(self.device, torch.float32).contiguous()

    def _inputs(self, x: torch.Tensor, target: torch.Tensor):
        x = self._x(x)
        if self.loss_name == "mse":
            check_rows(target, self.batch, self.widths[-1], "target")
            target = target.to(self.device, torch.float32).contiguous()
        else:
            if tuple(target.shape) != (self.batch,):
                raise RuntimeError(f"labels must be [{self.batch}], got {list(target.shape)}")
            # checked once per labels tensor and version (full-batch loops pass
            # the same tensor every step); the weak reference cannot outlive
            # the tensor, so a new tensor at a reused address is checked again
            seen = self._labels_checked
            if seen is None or seen[0]() is not target or seen[1] != target._version:
                check_labels(target, self.widths[-1])
                self._labels_checked = (weakref.ref(target), target._version)
            target = target.to(self.device, torch.int64).contiguous()
        return x, target

    def fit(self, x: torch.Tensor, target: torch.Tensor, steps: int) -> torch.Tensor:
        """``steps`` training steps on the same batch (the reference loop's
        full-batch epochs, README.md:61-69) issued in one library call;
        returns the per-step losses as a device tensor [steps]."""
        x, target = self._inputs(x, target)
        losses = torch.empty(int(steps), dtype=torch.float32, device=self.device)
        _lib.check(self._lib.ckan_exec_steps(self._h, x.data_ptr(), target.data_ptr(), int(steps),
                                             losses.data_ptr(), self._stream()))
        return losses

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self._x(x)
        y = torch.empty(self.batch, self.widths[-1], dtype=torch.float32, device=self.device)
        _lib.check(self._lib.ckan_exec_forward(self._h, x.data_ptr(), y.data_ptr(), self._stream()))
        return y

    def state_dict(self) -> dict:
        """Master coefficients (and Adam moments + step) for checkpointing."""
        sd = {"widths": list(self.widths), "degrees": list(self.degrees)}
        for l in range(len(self.degrees)):
            sd[f"{l}.cheby_coeffs"] = self.get_coeffs(l).cpu()
            if self.optimizer == "adam":
                m = torch.empty(self._shape(l), device=self.device)
                v = torch.empty(self._shape(l), device=self.device)
                st = ctypes.c_int64()
                _lib.check(self._lib.ckan_exec_get_adam_state(self._h, l, m.data_ptr(), v.data_ptr(),
                                                              ctypes.byref(st), self._stream()))
                sd[f"{l}.exp_avg"], sd[f"{l}.exp_avg_sq"], sd["step"] = m.cpu(), v.cpu(), st.value
        return sd

    def load_state_dict(self, sd: dict) -> None:
        for l in range(len(self.degrees)):
            self.set_coeffs(l, sd[f"{l}.cheby_coeffs"])
            if self.optimizer == "adam" and f"{l}.exp_avg" in sd:
                m = sd[f"{l}.exp_avg"].to(self.device, torch.float32).contiguous()
                v = sd[f"{l}.exp_avg_sq"].to(self.device, torch.float32).contiguous()
                _lib.check(self._lib.ckan_exec_set_adam_state(self._h, l, m.data_ptr(), v.data_ptr(),
                                                              int(sd["step"]), self._stream()))

    def close(self) -> None:
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.ckan_exec_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
