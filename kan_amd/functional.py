"""Autograd functions over the C-ABI: the ChebyKAN forward/backward and the
materialised basis.  Device memory and streams come from torch; all compute
is the HIP library's.  Tensors on the CPU are rejected: there is no CPU path.
"""
from __future__ import annotations

import ctypes
import threading
import weakref

import torch

from . import _lib

_COMPUTE = {"fp32": _lib.CKAN_COMPUTE_FP32, "bf16": _lib.CKAN_COMPUTE_BF16}

# Forward workspaces hold the split-K partial tiles of the small-batch paths
# (written before they are read, so never cleared).  One per (device,
# stream): calls sharing a workspace must not overlap in time.
_fwd_ws = {}
_fwd_ws_lock = threading.Lock()


def _forward_workspace(device: torch.device, nbytes: int, stream: int) -> torch.Tensor:
    key = (device.index, stream)
    with _fwd_ws_lock:
        ws = _fwd_ws.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
            _fwd_ws[key] = ws
    return ws


# Backward workspaces (the dy re-layouts, column-sum and split-K partials, all
# written before they are read) and their sizes: likewise one per (device,
# stream), and the size per (descriptor object, dx wanted, dC wanted).
_bwd_ws = {}
_bwd_sizes = {}


def _backward_workspace(device: torch.device, desc, need_dx: bool, need_dc: bool,
                        stream: int):
    # keyed by the descriptor object's id; the entry holds the object, so the
    # id cannot be reused while the entry lives
    skey = (id(desc), need_dx, need_dc)
    ent = _bwd_sizes.get(skey)
    if ent is None or ent[0] is not desc:
        ent = (desc, _lib.load().ckan_bwd_workspace_bytes(desc, int(need_dx), int(need_dc)))
        if len(_bwd_sizes) > 4096:
            _bwd_sizes.clear()
        _bwd_sizes[skey] = ent
    nbytes = ent[1]
    key = (device.index, stream)
    with _fwd_ws_lock:
        ws = _bwd_ws.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
            _bwd_ws[key] = ws
    return ws, nbytes


# Packed-operand cache.  The reference re-lays C out inside the einsum on every
# call (kan/basis/chebyshev.py:101); here the packed operands depend only on
# the coefficients' values and the layer's shape, precision and basis, so the
# last packing of each coefficient tensor is kept and reused while the tensor
# is unchanged: same object, same storage and the same version counter (every
# in-place update, an optimizer step included, advances it).  A changed tensor
# is packed into a new buffer, so a graph recorded before the change keeps its
# own operands for its backward.  Code that writes the coefficients through a
# raw pointer (a C-ABI call) must advance the version itself, as kan_amd.optim
# does (torch.autograd.graph.increment_version).  Entries die with their tensor; one packed
# buffer per live coefficient tensor stays allocated (2 I O P bytes in bf16,
# about 4 I O P in fp32).  clear_pack_cache() drops them all.
# Entries are keyed by id(tensor) and hold a weak reference to the tensor
# (checked by identity on lookup; a tensor's == is elementwise, so weak-keyed
# dictionaries cannot hold tensors) whose callback drops the entry.
_pack_cache = {}  # id(coeffs) -> (weakref to coeffs, key, packed)
_pack_lock = threading.Lock()


def clear_pack_cache() -> None:
    """Release every cached packed-coefficient buffer."""
    with _pack_lock:
        _pack_cache.clear()


def cached_pack(coeffs: torch.Tensor):
    """The packed buffer cached for ``coeffs`` (whatever its version), or None."""
    with _pack_lock:
        ent = _pack_cache.get(id(coeffs))
    return ent[2] if ent is not None and ent[0]() is coeffs else None


def _cache_get(coeffs: torch.Tensor, key):
    with _pack_lock:
        ent = _pack_cache.get(id(coeffs))
    if ent is not None and ent[0]() is coeffs and ent[1] == key:
        return ent[2]
    return None


def _cache_put(coeffs: torch.Tensor, key, packed: torch.Tensor) -> None:
    i = id(coeffs)

    def drop(ref, i=i):  # the tensor died: its entry goes (unless already replaced)
        ent = _pack_cache.get(i)
        if ent is not None and ent[0] is ref:
            _pack_cache.pop(i, None)

    with _pack_lock:
        _pack_cache[i] = (weakref.ref(coeffs, drop), key, packed)


def _pack_key(coeffs: torch.Tensor, compute: str, spec, affine):
    spec_key = None if spec is None else bytes(spec)
    return (coeffs._version, coeffs.data_ptr(), coeffs.dtype, tuple(coeffs.shape), coeffs.device,
            compute, spec_key, None if affine is None else tuple(affine))


def _require_device(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "kan_amd ChebyKAN runs only on a ROCm device (MI355X); got a tensor on "
                f"{t.device}. Move the module and inputs to 'cuda'.")


def compute_code(compute: str) -> int:
    try:
        return _COMPUTE[compute]
    except KeyError:
        raise ValueError(f"compute must be one of {sorted(_COMPUTE)}, got {compute!r}") from None


def coeff_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return _lib.CKAN_DTYPE_F32
    if dtype == torch.bfloat16:
        return _lib.CKAN_DTYPE_BF16
    raise RuntimeError(f"kan_amd ChebyKAN supports float32 or bfloat16 coefficients, got {dtype}")


# Descriptors and their tanh-cache and forward-workspace sizes by (batch, in,
# out, degree, compute, coefficient dtype, affine).
_descs = {}
# tanh caches of forwards that keep no graph (nothing reads them afterwards),
# one per (device, stream), grown as needed: calls sharing one must not overlap.
_t_scratch = {}


def _desc_sizes(batch, in_dim, out_dim, degree, compute, dtype, affine):
    """(desc, tanh-cache elements, forward workspace bytes), cached per shape:
    the two sizes are host-side functions of the descriptor alone."""
    key = (batch, in_dim, out_dim, degree, compute, dtype, affine)
    ent = _descs.get(key)
    if ent is None:
        d = _lib.make_desc(batch, in_dim, out_dim, degree, compute_code(compute), coeff_code(dtype),
                           affine)
        lib = _lib.load()
        ent = (d, lib.ckan_tcache_elems(d), lib.ckan_fwd_workspace_bytes(d))
        if len(_descs) > 4096:
            _descs.clear()
        _descs[key] = ent
    return ent


def _layer_forward(x, coeffs, compute, spec, affine, keep_t):
    """The layer's forward through the C-ABI: returns (y, t, packed, desc).
    With keep_t the tanh cache is a new tensor (saved for the backward);
    otherwise a per-stream scratch buffer."""
    _require_device(x, coeffs)
    if coeffs.dim() != 3:
        raise RuntimeError(f"coefficients must be [in, out, degree+1], got {tuple(coeffs.shape)}")
    in_dim, out_dim, dd = coeffs.shape
    if x.dim() != 2 or x.shape[1] != in_dim:
        raise RuntimeError(f"x must be [batch, {in_dim}], got {tuple(x.shape)}")
    lib = _lib.load()
    dev = x.device
    x32 = x.contiguous() if x.dtype == torch.float32 else x.float().contiguous()
    desc, t_elems, ws_bytes = _desc_sizes(x32.shape[0], in_dim, out_dim, dd - 1, compute,
                                          coeffs.dtype, None if affine is None else tuple(affine))
    stream = _lib.stream_ptr(dev)
    if keep_t:
        t = torch.empty(t_elems, dtype=torch.float32, device=dev)
    else:
        tkey = (dev.index, stream)
        t = _t_scratch.get(tkey)
        if t is None or t.numel() < t_elems:
            t = torch.empty(max(t_elems, 64), dtype=torch.float32, device=dev)
            _t_scratch[tkey] = t
    y = torch.empty(x32.shape[0], out_dim, dtype=torch.float32, device=dev)
    ws = _forward_workspace(dev, ws_bytes, stream) if ws_bytes else None
    key = _pack_key(coeffs, compute, spec, affine)
    packed = _cache_get(coeffs, key)
    if packed is not None:
        _lib.check(lib.ckan_forward(desc, x32.data_ptr(), packed.data_ptr(), y.data_ptr(),
                                    t.data_ptr(), _lib.ptr(ws), ws_bytes, stream))
    else:
        c = coeffs.detach().contiguous()
        packed = torch.empty(lib.ckan_packed_bytes(desc), dtype=torch.uint8, device=dev)
        # pack (in the family's basis when a spec is given) and forward in one call
        _lib.check(lib.ckan_pack_forward(desc, spec, c.data_ptr(), packed.data_ptr(),
                                         x32.data_ptr(), y.data_ptr(), t.data_ptr(),
                                         _lib.ptr(ws), ws_bytes, stream))
        _cache_put(coeffs, key, packed)
    return y, t, packed, desc


def _needs_graph(x: torch.Tensor, coeffs: torch.Tensor) -> bool:
    return torch.is_grad_enabled() and (x.requires_grad or coeffs.requires_grad)


class ChebyKANFunction(torch.autograd.Function):
    """y = einsum('bid,iod->bo', T(tanh x), C) with hand-written HIP backward.

    With a basis ``spec`` (``_lib.CkanBasisSpec``), C holds the coefficients
    of that family P_n(s tanh x) instead: the library packs C M (the same
    function in the Chebyshev basis) and maps the coefficient gradient back
    through M^T.
    """

    @staticmethod
    def forward(ctx, x: torch.Tensor, coeffs: torch.Tensor, compute: str = "fp32", spec=None,
                affine=None):
        y, t, packed, desc = _layer_forward(x, coeffs, compute, spec, affine, keep_t=True)
        ctx.save_for_backward(t, packed)
        ctx.desc = desc
        ctx.spec = spec
        ctx.x_dtype = x.dtype
        ctx.c_dtype = coeffs.dtype
        return y

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        t, packed = ctx.saved_tensors
        desc = ctx.desc
        need_dx, need_dc = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_dx or need_dc):
            return None, None, None, None, None
        lib = _lib.load()
        dev = dy.device
        dy32 = dy.contiguous() if dy.dtype == torch.float32 else dy.float().contiguous()
        dx = torch.empty(desc.batch, desc.in_dim, dtype=torch.float32, device=dev) if need_dx else None
        dc = (torch.empty(desc.in_dim, desc.out_dim, desc.degree + 1, dtype=torch.float32, device=dev)
              if need_dc else None)
        stream = _lib.stream_ptr(dev)
        ws, ws_bytes = _backward_workspace(dev, desc, need_dx, need_dc, stream)
        if ctx.spec is None:
            _lib.check(lib.ckan_backward(desc, t.data_ptr(), packed.data_ptr(), dy32.data_ptr(),
                                         _lib.ptr(dx), _lib.ptr(dc), 0, ws.data_ptr(), ws_bytes,
                                         stream))
        else:  # dC = dC' M^T, applied by the dC launch where it can
            _lib.check(lib.ckan_backward_basis(desc, ctx.spec, t.data_ptr(), packed.data_ptr(),
                                               dy32.data_ptr(), _lib.ptr(dx), _lib.ptr(dc),
                                               ws.data_ptr(), ws_bytes, stream))
        if dx is not None and ctx.x_dtype != torch.float32:
            dx = dx.to(ctx.x_dtype)
        if dc is not None and ctx.c_dtype != torch.float32:
            dc = dc.to(ctx.c_dtype)
        return dx, dc, None, None, None


class ChebyshevBasisFunction(torch.autograd.Function):
    """T_d(t) for d = 0..degree, materialised as [..., degree+1] (fp32)."""

    @staticmethod
    def forward(ctx, t: torch.Tensor, degree: int):
        _require_device(t)
        lib = _lib.load()
        t32 = t.contiguous() if t.dtype == torch.float32 else t.float().contiguous()
        out = torch.empty(*t32.shape, degree + 1, dtype=torch.float32, device=t.device)
        _lib.check(lib.ckan_basis(t32.data_ptr(), t32.numel(), int(degree), out.data_ptr(),
                                  _lib.stream_ptr(t.device)))
        ctx.save_for_backward(t32)
        ctx.degree = degree
        ctx.t_dtype = t.dtype
        return out

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        (t32,) = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None
        lib = _lib.load()
        g32 = g.contiguous() if g.dtype == torch.float32 else g.float().contiguous()
        dt = torch.empty_like(t32)
        _lib.check(lib.ckan_basis_backward(t32.data_ptr(), g32.data_ptr(), t32.numel(),
                                           int(ctx.degree), dt.data_ptr(),
                                           _lib.stream_ptr(t32.device)))
        return dt.to(ctx.t_dtype), None


class FamilyBasisFunction(torch.autograd.Function):
    """P_n(t) for n = 0..degree of a recurrence family, materialised (fp32)."""

    @staticmethod
    def forward(ctx, t: torch.Tensor, spec):
        _require_device(t)
        lib = _lib.load()
        t32 = t.contiguous() if t.dtype == torch.float32 else t.float().contiguous()
        out = torch.empty(*t32.shape, spec.degree + 1, dtype=torch.float32, device=t.device)
        _lib.check(lib.ckan_family_basis(spec, t32.data_ptr(), t32.numel(), out.data_ptr(),
                                         _lib.stream_ptr(t.device)))
        ctx.save_for_backward(t32)
        ctx.spec = spec
        ctx.t_dtype = t.dtype
        return out

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        (t32,) = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None
        lib = _lib.load()
        g32 = g.contiguous() if g.dtype == torch.float32 else g.float().contiguous()
        dt = torch.empty_like(t32)
        _lib.check(lib.ckan_family_basis_backward(ctx.spec, t32.data_ptr(), g32.data_ptr(),
                                                  t32.numel(), dt.data_ptr(),
                                                  _lib.stream_ptr(t32.device)))
        return dt.to(ctx.t_dtype), None


# fp64 recurrence blocks of basis families, by (device, spec bytes): a few
# hundred bytes each, written once (ckan_write_recurrence_f64).
_rec64 = {}
_rec64_lock = threading.Lock()


def _recurrence_f64(spec, device: torch.device) -> torch.Tensor:
    key = (device, bytes(spec))
    with _rec64_lock:
        rec = _rec64.get(key)
    if rec is None:
        lib = _lib.load()
        nbytes = lib.ckan_recurrence_bytes_f64(spec)
        if nbytes == 0:
            raise RuntimeError(f"kan_amd: basis degree {spec.degree} is outside the fp64 path's 0..1024")
        rec = torch.empty(nbytes // 8, dtype=torch.float64, device=device)
        _lib.check(lib.ckan_write_recurrence_f64(spec, rec.data_ptr(), _lib.stream_ptr(device)))
        with _rec64_lock:
            _rec64[key] = rec
    return rec


class ChebyKANFunction64(torch.autograd.Function):
    """The layer in fp64 end to end (the reference's behaviour for fp64
    parameters): x is taken as fp64, y, dx and dC are fp64.  With a basis
    ``spec`` the basis is that family's P_n(s tanh x), by its recurrence in
    fp64 (the Jacobi and Hermite layers after .double())."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, coeffs: torch.Tensor, spec=None):
        _require_device(x, coeffs)
        if coeffs.dim() != 3:
            raise RuntimeError(f"coefficients must be [in, out, degree+1], got {tuple(coeffs.shape)}")
        in_dim, out_dim, dd = coeffs.shape
        if x.dim() != 2 or x.shape[1] != in_dim:
            raise RuntimeError(f"x must be [batch, {in_dim}], got {tuple(x.shape)}")
        lib = _lib.load()
        dev = x.device
        x64 = x.contiguous() if x.dtype == torch.float64 else x.double().contiguous()
        c = coeffs.detach().contiguous()
        desc = _lib.make_desc(x64.shape[0], in_dim, out_dim, dd - 1, 0, 0)
        t = torch.empty(x64.shape[0], in_dim, dtype=torch.float64, device=dev)
        y = torch.empty(x64.shape[0], out_dim, dtype=torch.float64, device=dev)
        rec = _recurrence_f64(spec, dev) if spec is not None else None
        if rec is None:
            _lib.check(lib.ckan_forward_f64(desc, x64.data_ptr(), c.data_ptr(), y.data_ptr(),
                                            t.data_ptr(), _lib.stream_ptr(dev)))
        else:
            _lib.check(lib.ckan_forward_f64_basis(desc, rec.data_ptr(), x64.data_ptr(), c.data_ptr(),
                                                  y.data_ptr(), t.data_ptr(), _lib.stream_ptr(dev)))
        ctx.save_for_backward(t, c, rec)
        ctx.desc = desc
        ctx.x_dtype = x.dtype
        return y

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        t, c, rec = ctx.saved_tensors
        desc = ctx.desc
        need_dx, need_dc = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_dx or need_dc):
            return None, None, None
        lib = _lib.load()
        dev = dy.device
        dy64 = dy.contiguous() if dy.dtype == torch.float64 else dy.double().contiguous()
        dx = torch.empty(desc.batch, desc.in_dim, dtype=torch.float64, device=dev) if need_dx else None
        dc = (torch.empty(desc.in_dim, desc.out_dim, desc.degree + 1, dtype=torch.float64, device=dev)
              if need_dc else None)
        if rec is None:
            _lib.check(lib.ckan_backward_f64(desc, t.data_ptr(), c.data_ptr(), dy64.data_ptr(),
                                             _lib.ptr(dx), _lib.ptr(dc), 0, _lib.stream_ptr(dev)))
        else:
            _lib.check(lib.ckan_backward_f64_basis(desc, rec.data_ptr(), t.data_ptr(), c.data_ptr(),
                                                   dy64.data_ptr(), _lib.ptr(dx), _lib.ptr(dc), 0,
                                                   _lib.stream_ptr(dev)))
        if dx is not None and ctx.x_dtype != torch.float64:
            dx = dx.to(ctx.x_dtype)
        return dx, dc, None


def chebykan(x: torch.Tensor, coeffs: torch.Tensor, compute: str = "fp32") -> torch.Tensor:
    """Functional ChebyKAN layer: x [B, in], coeffs [in, out, D] -> y [B, out].

    fp64 coefficients select the fp64 path (``compute`` does not apply there)."""
    if coeffs.dtype == torch.float64:
        return ChebyKANFunction64.apply(x, coeffs)
    if not _needs_graph(x, coeffs):  # inference: no autograd node, no tanh cache kept
        return _layer_forward(x, coeffs, compute, None, None, keep_t=False)[0]
    return ChebyKANFunction.apply(x, coeffs, compute, None)


def family_kan(x: torch.Tensor, coeffs: torch.Tensor, spec, compute: str = "fp32",
               affine=None) -> torch.Tensor:
    """y = einsum('bid,iod->bo', P(s u), C) for the family of ``spec``, with
    u = tanh x, or u = affine[0] x + affine[1] when ``affine`` is given."""
    if coeffs.dtype == torch.float64:
        if affine is not None:
            raise RuntimeError("kan_amd: a Hermite layer with a finite domain (an affine input map) "
                               "runs in float32 or bfloat16; its fp64 path takes the tanh map only")
        return ChebyKANFunction64.apply(x, coeffs, spec)
    if not _needs_graph(x, coeffs):
        return _layer_forward(x, coeffs, compute, spec, affine, keep_t=False)[0]
    return ChebyKANFunction.apply(x, coeffs, compute, spec, affine)


def family_basis(t: torch.Tensor, spec) -> torch.Tensor:
    return FamilyBasisFunction.apply(t, spec)


def chebyshev_basis(t: torch.Tensor, degree: int) -> torch.Tensor:
    return ChebyshevBasisFunction.apply(t, degree)


# ---- derivatives with respect to the input (kan/layers/base.py:102-141) ------

def _spec_ref(spec):
    return None if spec is None else ctypes.byref(spec)


def _derivative_desc(coeffs: torch.Tensor, batch: int = 0, affine=None) -> "_lib.CkanDesc":
    in_dim, out_dim, dd = coeffs.shape
    return _lib.make_desc(batch, in_dim, out_dim, dd - 1, _lib.CKAN_COMPUTE_FP32, _lib.CKAN_DTYPE_F32,
                          None if affine is None else tuple(affine))


def _f32_coeffs(coeffs: torch.Tensor) -> torch.Tensor:
    _require_device(coeffs)
    if coeffs.dim() != 3:
        raise RuntimeError(f"coefficients must be [in, out, degree+1], got {tuple(coeffs.shape)}")
    if coeffs.dtype == torch.float64:
        raise RuntimeError("kan_amd derivatives take float32 (or bfloat16) coefficients; the fp64 "
                           "path serves the forward and backward only")
    return coeffs.float().contiguous()


class DerivativeCoeffsFunction(torch.autograd.Function):
    """Ck = C R [in, out, D + order]: the Chebyshev coefficients in tanh x (in
    u = affine[0] x + affine[1] under an affine input map) of the order-k
    x-derivative of each univariate function (R from the library, exact in
    fp64, applied in fp32); backward dC = dCk R^T."""

    @staticmethod
    def forward(ctx, coeffs: torch.Tensor, spec, order: int, affine=None):
        c = _f32_coeffs(coeffs.detach())
        in_dim, out_dim, dd = c.shape
        out = torch.empty(in_dim, out_dim, dd + order, dtype=torch.float32, device=c.device)
        desc = _derivative_desc(c, 0, affine)
        lib = _lib.load()
        _lib.check(lib.ckan_derivative_coeffs(desc, _spec_ref(spec), int(order), c.data_ptr(),
                                              out.data_ptr(), _lib.stream_ptr(c.device)))
        ctx.desc, ctx.spec, ctx.order, ctx.c_dtype = desc, spec, order, coeffs.dtype
        return out

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        g = g.float().contiguous()
        d = ctx.desc
        dc = torch.empty(d.in_dim, d.out_dim, d.degree + 1, dtype=torch.float32, device=g.device)
        lib = _lib.load()
        _lib.check(lib.ckan_derivative_coeffs_backward(d, _spec_ref(ctx.spec), int(ctx.order),
                                                       g.data_ptr(), dc.data_ptr(),
                                                       _lib.stream_ptr(g.device)))
        if ctx.c_dtype != torch.float32:
            dc = dc.to(ctx.c_dtype)
        return dc, None, None, None


def derivative_coeffs(coeffs: torch.Tensor, spec, order: int, affine=None) -> torch.Tensor:
    return DerivativeCoeffsFunction.apply(coeffs, spec, int(order), affine)


def derivatives(x: torch.Tensor, coeffs: torch.Tensor, spec, order: int = 1,
                compute: str = "fp32", affine=None) -> torch.Tensor:
    """[B, out]: sum_i d^order f_{i,o} / dx^order (x[b, i]), the sum over inputs of
    each univariate function's order-th x-derivative (differentiable in x and C).
    ``affine`` = (a, b): the layer maps x by u = a x + b instead of tanh."""
    if order < 0:
        raise ValueError(f"order must be >= 0, got {order}")
    if order == 0:
        if spec is None and affine is None:
            return chebykan(x, coeffs, compute)
        if spec is None:
            return ChebyKANFunction.apply(x, coeffs, compute, None, affine)
        return family_kan(x, coeffs, spec, compute, affine)
    return ChebyKANFunction.apply(x, derivative_coeffs(coeffs, spec, order, affine), compute, None,
                                  affine)


def jacobian(x: torch.Tensor, coeffs: torch.Tensor, spec, affine=None) -> torch.Tensor:
    """[B, out, in]: d y[b, o] / d x[b, i] (fp32; not differentiable); ``affine``
    as in derivatives."""
    c = _f32_coeffs(coeffs.detach())
    _require_device(x)
    in_dim, out_dim, _ = c.shape
    if x.dim() != 2 or x.shape[1] != in_dim:
        raise RuntimeError(f"x must be [batch, {in_dim}], got {tuple(x.shape)}")
    x32 = x.detach().float().contiguous()
    desc = _derivative_desc(c, x32.shape[0], affine)
    lib = _lib.load()
    jac = torch.empty(x32.shape[0], out_dim, in_dim, dtype=torch.float32, device=x.device)
    ws_bytes = lib.ckan_jacobian_workspace_bytes(desc)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=x.device)
    _lib.check(lib.ckan_jacobian(desc, _spec_ref(spec), x32.data_ptr(), c.data_ptr(),
                                 jac.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream_ptr(x.device)))
    return jac
