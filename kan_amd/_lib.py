"""ctypes binding of the C-ABI in include/chebykan.h.

The library is the in-tree ``kan_amd/libckan_gfx950.so`` built by
``kan_amd.build``.  torch is imported first so that the HIP runtime the
library resolves (soname libamdhip64.so.7) is the one torch already loaded;
streams and device pointers handed over from torch are then valid in it.
There is no fallback: if the library is missing or cannot be loaded, every
entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libckan_gfx950.so")

CKAN_OK = 0
CKAN_ERR_INVALID_ARG = 1
CKAN_ERR_UNSUPPORTED = 2
CKAN_ERR_WORKSPACE = 3
CKAN_ERR_HIP = 4
# size of the fixed device scratch of ckan_forward_noalloc (include/chebykan.h)
CKAN_NOALLOC_SCRATCH_BYTES = 16 << 20

CKAN_COMPUTE_FP32 = 0
CKAN_COMPUTE_BF16 = 1
CKAN_DTYPE_F32 = 0
CKAN_DTYPE_BF16 = 1


class CkanDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("in_dim", ctypes.c_int32),
        ("out_dim", ctypes.c_int32),
        ("degree", ctypes.c_int32),
        ("compute", ctypes.c_int32),
        ("coeff_dtype", ctypes.c_int32),
        ("input_map", ctypes.c_int32),
        ("in_scale", ctypes.c_float),
        ("in_shift", ctypes.c_float),
    ]


CKAN_INPUT_TANH = 0
CKAN_INPUT_AFFINE = 1


CKAN_BASIS_CHEBYSHEV = 0
CKAN_BASIS_JACOBI = 1
CKAN_BASIS_HERMITE = 2
CKAN_BASIS_HERMITE_E = 3


class CkanBasisSpec(ctypes.Structure):
    _fields_ = [
        ("family", ctypes.c_int32),
        ("degree", ctypes.c_int32),
        ("alpha", ctypes.c_double),
        ("beta", ctypes.c_double),
        ("scale", ctypes.c_double),
    ]


def make_spec(family: int, degree: int, alpha: float = 0.0, beta: float = 0.0,
              scale: float = 1.0) -> CkanBasisSpec:
    return CkanBasisSpec(int(family), int(degree), float(alpha), float(beta), float(scale))


class CkanError(RuntimeError):
    """Raised when a C-ABI call returns a non-zero ckan_status."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[ckan status {code}] {msg}")
        self.code = code


_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_pdesc = ctypes.POINTER(CkanDesc)
_pspec = ctypes.POINTER(CkanBasisSpec)

# name -> (restype, argtypes); every function declared in include/chebykan.h
SIGNATURES = {
    "ckan_packed_bytes": (_sz, [_pdesc]),
    "ckan_tcache_elems": (_sz, [_pdesc]),
    "ckan_fwd_workspace_bytes": (_sz, [_pdesc]),
    "ckan_bwd_workspace_bytes": (_sz, [_pdesc, ctypes.c_int, ctypes.c_int]),
    "ckan_workspace_init": (ctypes.c_int, [_vp, _sz, _vp]),
    "ckan_pack_coeffs": (ctypes.c_int, [_pdesc, _vp, _vp, _vp]),
    "ckan_forward": (ctypes.c_int, [_pdesc, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ckan_forward_noalloc": (ctypes.c_int, [_pdesc, _vp, _vp, _vp, _vp, _vp]),
    "ckan_pack_forward": (ctypes.c_int, [_pdesc, _pspec, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ckan_backward": (ctypes.c_int, [_pdesc, _vp, _vp, _vp, _vp, _vp, ctypes.c_int, _vp, _sz, _vp]),
    "ckan_forward_f64": (ctypes.c_int, [_pdesc, _vp, _vp, _vp, _vp, _vp]),
    "ckan_backward_f64": (ctypes.c_int, [_pdesc, _vp, _vp, _vp, _vp, _vp, ctypes.c_int, _vp]),
    "ckan_recurrence_bytes_f64": (_sz, [_pspec]),
    "ckan_write_recurrence_f64": (ctypes.c_int, [_pspec, _vp, _vp]),
    "ckan_forward_f64_basis": (ctypes.c_int, [_pdesc, _vp, _vp, _vp, _vp, _vp, _vp]),
    "ckan_backward_f64_basis": (ctypes.c_int, [_pdesc, _vp, _vp, _vp, _vp, _vp, _vp, ctypes.c_int,
                                               _vp]),
    "ckan_basis_to_chebyshev": (ctypes.c_int, [_pspec, ctypes.POINTER(_f64)]),
    "ckan_pack_coeffs_basis": (ctypes.c_int, [_pdesc, _pspec, _vp, _vp, _vp]),
    "ckan_coeff_grad_from_chebyshev": (ctypes.c_int, [_pdesc, _pspec, _vp, _vp, ctypes.c_int, _vp]),
    "ckan_backward_basis": (ctypes.c_int, [_pdesc, _pspec, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ckan_family_basis": (ctypes.c_int, [_pspec, _vp, _i64, _vp, _vp]),
    "ckan_family_basis_backward": (ctypes.c_int, [_pspec, _vp, _vp, _i64, _vp, _vp]),
    "ckan_derivative_matrix": (ctypes.c_int, [_pspec, _i32, _i32, ctypes.POINTER(_f64)]),
    "ckan_derivative_coeffs": (ctypes.c_int, [_pdesc, _pspec, _i32, _vp, _vp, _vp]),
    "ckan_derivative_coeffs_backward": (ctypes.c_int, [_pdesc, _pspec, _i32, _vp, _vp, _vp]),
    "ckan_jacobian_workspace_bytes": (_sz, [_pdesc]),
    "ckan_jacobian": (ctypes.c_int, [_pdesc, _pspec, _vp, _vp, _vp, _vp, _sz, _vp]),
    "ckan_basis": (ctypes.c_int, [_vp, _i64, _i32, _vp, _vp]),
    "ckan_basis_backward": (ctypes.c_int, [_vp, _vp, _i64, _i32, _vp, _vp]),
    "ckan_sgd_step": (ctypes.c_int, [_vp, _vp, _i64, _f32, _f32, _vp]),
    "ckan_adam_step": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _f64, _f64, _f64, _f64, _f64, _vp]),
    "ckan_last_error": (ctypes.c_char_p, []),
    "ckan_version": (ctypes.c_char_p, []),
    "ckan_profile_enable": (ctypes.c_int, [ctypes.c_int]),
    "ckan_profile_report": (_sz, [ctypes.c_char_p, _sz]),
}

class CkanExecConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", ctypes.c_int32),
        ("widths", ctypes.POINTER(ctypes.c_int32)),
        ("degrees", ctypes.POINTER(ctypes.c_int32)),
        ("batch", ctypes.c_int64),
        ("compute", ctypes.c_int32),
        ("loss", ctypes.c_int32),
        ("optimizer", ctypes.c_int32),
        ("use_graph", ctypes.c_int32),
        ("lr", ctypes.c_float),
        ("beta1", ctypes.c_float),
        ("beta2", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("weight_decay", ctypes.c_float),
        ("flags", ctypes.c_int32),
    ]


CKAN_EXEC_NO_FUSED_SMALL = 1
CKAN_EXEC_PACK_EACH_STEP = 2


CKAN_LOSS_MSE = 0
CKAN_LOSS_CE = 1
CKAN_OPT_SGD = 0
CKAN_OPT_ADAM = 1

_pcfg = ctypes.POINTER(CkanExecConfig)
SIGNATURES.update({
    "ckan_exec_create": (ctypes.c_int, [_pcfg, ctypes.POINTER(_vp), _vp]),
    "ckan_exec_create_basis": (ctypes.c_int, [_pcfg, _pspec, ctypes.POINTER(_f32),
                                              ctypes.POINTER(_vp), _vp]),
    "ckan_exec_destroy": (ctypes.c_int, [_vp]),
    "ckan_exec_set_coeffs": (ctypes.c_int, [_vp, _i32, _vp, _vp]),
    "ckan_exec_get_coeffs": (ctypes.c_int, [_vp, _i32, _vp, _vp]),
    "ckan_exec_get_adam_state": (ctypes.c_int, [_vp, _i32, _vp, _vp, ctypes.POINTER(_i64), _vp]),
    "ckan_exec_set_adam_state": (ctypes.c_int, [_vp, _i32, _vp, _vp, _i64, _vp]),
    "ckan_exec_step": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "ckan_exec_forward": (ctypes.c_int, [_vp, _vp, _vp, _vp]),
    "ckan_exec_steps": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _vp]),
})

_lib = None
_lock = threading.Lock()


def load():
    """Load (once) and return the C-ABI library; raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"kan_amd: HIP library {LIB_PATH} is not built; run `python -m kan_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc: int) -> None:
    if rc != CKAN_OK:
        msg = load().ckan_last_error().decode(errors="replace")
        raise CkanError(rc, msg)


def make_desc(batch: int, in_dim: int, out_dim: int, degree: int, compute: int,
              coeff_dtype: int, affine=None) -> CkanDesc:
    """``affine`` = (scale, shift) selects the input map t = scale * x + shift
    instead of tanh(x)."""
    if affine is None:
        return CkanDesc(int(batch), int(in_dim), int(out_dim), int(degree), int(compute),
                        int(coeff_dtype), CKAN_INPUT_TANH, 0.0, 0.0)
    return CkanDesc(int(batch), int(in_dim), int(out_dim), int(degree), int(compute),
                    int(coeff_dtype), CKAN_INPUT_AFFINE, float(affine[0]), float(affine[1]))


def stream_ptr(device: torch.device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()


def profile_enable(on: bool) -> None:
    check(load().ckan_profile_enable(1 if on else 0))


def derivative_matrix(spec, degree: int, order: int):
    """R [degree+1, degree+1+order] (fp64, host): the Chebyshev coefficients in
    t = tanh x of d^order/dx^order P_n(s tanh x) (spec None: T_n(tanh x))."""
    import numpy as np
    out = np.zeros((degree + 1) * (degree + 1 + order), dtype=np.float64)
    sp = None if spec is None else ctypes.byref(spec)
    check(load().ckan_derivative_matrix(sp, int(degree), int(order),
                                        out.ctypes.data_as(ctypes.POINTER(_f64))))
    return out.reshape(degree + 1, degree + 1 + order)


def profile_report() -> dict:
    """{kernel name: (launch count, total ms)} of the launches since the last report."""
    lib = load()
    buf = ctypes.create_string_buffer(1 << 16)  # the report clears the records: call once
    lib.ckan_profile_report(buf, len(buf))
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, ms = line.split()
        out[name] = (int(cnt), float(ms))
    return out
