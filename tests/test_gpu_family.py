"""GPU parity of the Jacobi / Hermite layers (HIP path through the C-ABI)
against the CPU oracle oracle/family_oracle.py.

Tolerances (norm-wise, ||a - b|| / ||b||), as for the Chebyshev layer:
  fp32 MFMA path:  1e-5 for y, dx and dC
  bf16 MFMA path:  2e-2
"""
import ctypes

import pytest
import torch

from kan_amd import _lib
from oracle import family_oracle as fo

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    n = b.norm().item()
    return (a - b).norm().item() / (n if n > 0 else 1.0)


def _spec(family, deg, alpha=0.0, beta=0.0):
    if family == "jacobi":
        return _lib.make_spec(_lib.CKAN_BASIS_JACOBI, deg, alpha, beta, 1.0)
    fam = _lib.CKAN_BASIS_HERMITE if family == "hermite" else _lib.CKAN_BASIS_HERMITE_E
    return _lib.make_spec(fam, deg, 0.0, 0.0, 3.0)


CASES = [
    # family, alpha, beta, B, I, O, deg
    ("jacobi", 0.0, 0.0, 256, 64, 48, 8),
    ("jacobi", 1.5, 0.5, 300, 40, 70, 3),
    ("jacobi", -0.5, 0.25, 2048, 256, 128, 8),   # pipelined forward (B > 512)
    ("jacobi", 2.0, 3.0, 16, 512, 96, 5),        # coefficient-streaming forward (B <= 64)
    ("hermite", 0, 0, 129, 64, 96, 16),
    ("hermite", 0, 0, 7, 5, 3, 1),
    ("hermite_e", 0, 0, 200, 72, 50, 12),
    ("hermite_e", 0, 0, 1024, 128, 256, 4),
    ("jacobi", 0.5, -0.25, 256, 1024, 1024, 8),  # one unsplit dC launch maps dC' M^T itself
    ("hermite", 0, 0, 128, 2048, 1024, 4),       # the same at degree 4 (256 outputs per block)
]


@pytest.mark.parametrize("compute,tol", [("fp32", FP32_TOL), ("bf16", BF16_TOL)])
@pytest.mark.parametrize("family,alpha,beta,B,I,O,deg", CASES)
def test_family_layer_forward_backward_parity(family, alpha, beta, B, I, O, deg, compute, tol):
    from kan_amd import functional as F
    print(f"{family}({alpha},{beta}) {compute} B={B} I={I} O={O} deg={deg}", flush=True)
    g = torch.Generator().manual_seed(B + I + deg)
    x = torch.randn(B, I, generator=g) * 1.5
    c = torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))
    dy = torch.randn(B, O, generator=g)
    y_ref, dx_ref, dc_ref = fo.family_forward_backward(x, c, dy, family, alpha, beta)
    xd = x.cuda().requires_grad_(True)
    cd = c.cuda().requires_grad_(True)
    y = F.family_kan(xd, cd, _spec(family, deg, alpha, beta), compute)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    assert _rel(y, y_ref) <= tol
    assert _rel(xd.grad, dx_ref) <= tol
    assert _rel(cd.grad, dc_ref) <= tol


def test_family_layers_through_module_api():
    import kan_amd
    torch.manual_seed(0)
    jl = kan_amd.JacobiKANLayer(64, 32, 6, alpha=0.5, beta=-0.25).cuda()
    hl = kan_amd.HermiteKANLayer(32, 10, 5, scaling="physicist").cuda()
    model = kan_amd.KANSequential(jl, hl)
    x = torch.randn(96, 64)
    y = model(x.cuda())
    y.sum().backward()
    torch.cuda.synchronize()
    cj = jl.jacobi_coeffs.detach().cpu().requires_grad_(True)
    ch = hl.hermite_coeffs.detach().cpu().requires_grad_(True)
    h1 = fo.family_forward(x, cj, "jacobi", 0.5, -0.25)
    y_ref = fo.family_forward(h1, ch, "hermite")
    y_ref.sum().backward()
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(jl.jacobi_coeffs.grad, cj.grad) <= FP32_TOL
    assert _rel(hl.hermite_coeffs.grad, ch.grad) <= FP32_TOL
    # a second backward accumulates into .grad
    g1 = jl.jacobi_coeffs.grad.clone()
    model(x.cuda()).sum().backward()
    torch.cuda.synchronize()
    assert _rel(jl.jacobi_coeffs.grad, 2 * g1) <= FP32_TOL


@pytest.mark.parametrize("family,alpha,beta", [("jacobi", 1.0, 0.5), ("hermite", 0, 0),
                                               ("hermite_e", 0, 0)])
def test_family_basis_functions_and_backward(family, alpha, beta):
    from kan_amd import functional as F
    deg = 9
    s = 1.0 if family == "jacobi" else 3.0
    t = (torch.rand(300, 7, generator=torch.Generator().manual_seed(1)) * 2 - 1) * s
    g = torch.randn(300, 7, deg + 1, generator=torch.Generator().manual_seed(2))
    tr = t.clone().double().requires_grad_(True)
    ref = fo.family_basis(tr, family, deg, alpha, beta)
    (ref * g.double()).sum().backward()
    td = t.cuda().requires_grad_(True)
    out = F.family_basis(td, _spec(family, deg, alpha, beta))
    (out * g.cuda()).sum().backward()
    torch.cuda.synchronize()
    assert _rel(out, ref) <= FP32_TOL
    assert _rel(td.grad, tr.grad) <= FP32_TOL


@pytest.mark.parametrize("I,O,deg", [(37, 19, 7), (5, 7, 8), (300, 260, 16)])
def test_coeff_grad_transform_accumulates(I, O, deg):
    """dC (+)= dC' M^T through the C-ABI, against the same product on the CPU
    (float4 blocks, a scalar tail of odd length, and a partial last block)."""
    import numpy as np
    lib = _lib.load()
    spec = _spec("hermite", deg)
    M = (ctypes.c_double * ((deg + 1) ** 2))()
    assert lib.ckan_basis_to_chebyshev(spec, M) == 0
    Mn = torch.tensor(np.array(M[:]).reshape(deg + 1, deg + 1))
    g = torch.Generator().manual_seed(4)
    dcheb = torch.randn(I, O, deg + 1, generator=g)
    base = torch.randn(I, O, deg + 1, generator=g)
    d = _lib.make_desc(1, I, O, deg, 0, 0)
    out = base.cuda()
    st = _lib.stream_ptr(out.device)
    dch = dcheb.cuda()
    _lib.check(lib.ckan_coeff_grad_from_chebyshev(d, spec, dch.data_ptr(), out.data_ptr(), 1, st))
    expect = base.double() + torch.einsum("iok,nk->ion", dcheb.double(), Mn)
    assert _rel(out, expect) <= FP32_TOL
    inplace = dcheb.cuda()
    _lib.check(lib.ckan_coeff_grad_from_chebyshev(d, spec, inplace.data_ptr(), inplace.data_ptr(), 0, st))
    torch.cuda.synchronize()
    assert _rel(inplace, torch.einsum("iok,nk->ion", dcheb.double(), Mn)) <= FP32_TOL


@pytest.mark.parametrize("compute,tol", [("fp32", FP32_TOL), ("bf16", BF16_TOL)])
@pytest.mark.parametrize("scaling,B,I,O,deg", [
    ("physicist", 300, 40, 70, 6),       # small-batch forward (split partials)
    ("probabilist", 2048, 256, 128, 8),  # pipelined forward, tanh stage replaced in the pack launch
    ("physicist", 20, 512, 64, 5),       # coefficient-streaming forward (affine map in the stream kernel)
    ("probabilist", 1000, 100, 150, 12),  # padded inputs: the separate input-map launch
])
def test_hermite_finite_domain_affine_map(scaling, B, I, O, deg, compute, tol):
    """HermiteKANLayer(domain=(lo, hi), normalize_domain=True) maps x linearly
    onto [-3, 3] (kan/basis/hermite.py:102-112) instead of 3 tanh(x): y, dx
    (chain factor 6 / (hi - lo)) and dC against the oracle, with some x outside
    the domain."""
    import kan_amd
    print(f"hermite affine {scaling} {compute} B={B} I={I} O={O} deg={deg}", flush=True)
    dom = (-2.0, 5.0)
    torch.manual_seed(B + deg)
    m = kan_amd.HermiteKANLayer(I, O, deg, scaling=scaling, domain=dom, normalize_domain=True,
                                compute=compute)
    c = m.hermite_coeffs.detach().clone()
    g = torch.Generator().manual_seed(B + I)
    # [-2.5, 5.5): partly outside [lo, hi], where |u| > 1 and T_k(u) grows
    # like cosh(k acosh |u|) (bf16 rounding grows with it)
    x = torch.rand(B, I, generator=g) * 8 - 2.5
    dy = torch.randn(B, O, generator=g)
    fam = "hermite" if scaling == "physicist" else "hermite_e"
    c_ref = c  # the bf16 path rounds C M (the Chebyshev-basis coefficients), as for the tanh map
    y_ref, dx_ref, dc_ref = fo.family_forward_backward(x, c_ref, dy, fam, domain=dom)
    m = m.cuda()
    xd = x.cuda().requires_grad_(True)
    y = m(xd)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    assert _rel(y, y_ref) <= tol
    assert _rel(xd.grad, dx_ref) <= tol
    assert _rel(m.hermite_coeffs.grad, dc_ref) <= tol
    # the tanh map would give a different function
    y_tanh = fo.family_forward(x, c_ref, fam)
    assert _rel(y, y_tanh) > 10 * tol


@pytest.mark.parametrize("family,compute,B,I,O,deg,fused", [
    ("jacobi", "bf16", 512, 1024, 1024, 8, True),     # one unsplit pipelined dC launch maps dC
    ("hermite", "fp32", 256, 2048, 1024, 4, True),     # degree 4: 256 outputs per block
    ("hermite_e", "bf16", 256, 1024, 1024, 12, True),  # degree 16, one stage group
    ("jacobi", "bf16", 2048, 256, 128, 8, False),     # split dC: the map is its own launch
    ("hermite", "fp32", 64, 64, 48, 5, False),        # small dC on the vector ALU
])
def test_backward_basis_equals_backward_then_map(family, compute, B, I, O, deg, fused):
    """ckan_backward_basis gives the bits of ckan_backward followed by the
    in-place ckan_coeff_grad_from_chebyshev, for dx and dC, and launches no
    separate map where one dC launch writes the whole gradient."""
    print(f"backward_basis {family} {compute} B={B} I={I} O={O} deg={deg}", flush=True)
    lib = _lib.load()
    spec = _spec(family, deg, 0.5, -0.25)
    cc = _lib.CKAN_COMPUTE_BF16 if compute == "bf16" else _lib.CKAN_COMPUTE_FP32
    d = _lib.make_desc(B, I, O, deg, cc, _lib.CKAN_DTYPE_F32)
    g = torch.Generator().manual_seed(B + I + deg)
    x = (torch.rand(B, I, generator=g) * 4 - 2).cuda()
    C = (torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))).cuda()
    dy = torch.randn(B, O, generator=g).cuda()
    st = _lib.stream_ptr(x.device)
    packed = torch.empty(lib.ckan_packed_bytes(d), dtype=torch.uint8, device=x.device)
    t = torch.empty(lib.ckan_tcache_elems(d), device=x.device)
    y = torch.empty(B, O, device=x.device)
    fwb = lib.ckan_fwd_workspace_bytes(d)
    fws = torch.empty(max(fwb, 256), dtype=torch.uint8, device=x.device)
    _lib.check(lib.ckan_pack_coeffs_basis(d, spec, C.data_ptr(), packed.data_ptr(), st))
    _lib.check(lib.ckan_forward(d, x.data_ptr(), packed.data_ptr(), y.data_ptr(), t.data_ptr(),
                                fws.data_ptr(), fwb, st))
    bwb = lib.ckan_bwd_workspace_bytes(d, 1, 1)
    ws = torch.empty(max(bwb, 256), dtype=torch.uint8, device=x.device)
    dx1, dc1 = torch.empty(B, I, device=x.device), torch.empty(I, O, deg + 1, device=x.device)
    _lib.check(lib.ckan_backward(d, t.data_ptr(), packed.data_ptr(), dy.data_ptr(), dx1.data_ptr(),
                                 dc1.data_ptr(), 0, ws.data_ptr(), bwb, st))
    _lib.check(lib.ckan_coeff_grad_from_chebyshev(d, spec, dc1.data_ptr(), dc1.data_ptr(), 0, st))
    dx2, dc2 = torch.full_like(dx1, float("nan")), torch.full_like(dc1, float("nan"))
    torch.cuda.synchronize()
    _lib.profile_enable(True)
    try:
        _lib.check(lib.ckan_backward_basis(d, spec, t.data_ptr(), packed.data_ptr(), dy.data_ptr(),
                                           dx2.data_ptr(), dc2.data_ptr(), ws.data_ptr(), bwb, st))
        torch.cuda.synchronize()
        rep = _lib.profile_report()
    finally:
        _lib.profile_enable(False)
    assert ("coeff_from_cheb" not in rep) == fused, rep
    assert torch.equal(dx1, dx2)
    assert torch.equal(dc1, dc2)
    assert dc1.abs().sum() > 0
