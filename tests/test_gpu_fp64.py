"""GPU parity of the fp64 path (ckan_forward_f64 / ckan_backward_f64) against
the oracle run in fp64: the reference layer with fp64 parameters computes in
fp64 (kan/layers/chebykan.py:48-51, kan/basis/chebyshev.py:78-101).

Tolerance: 1e-11 norm-wise relative for y, dx and dC (both sides fp64; they
differ only in summation order and in acos/cos versus the recurrence)."""
import pytest
import torch

from oracle import chebykan_oracle as orc

pytestmark = pytest.mark.gpu

FP64_TOL = 1e-11


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    n = b.norm().item()
    return (a - b).norm().item() / (n if n > 0 else 1.0)


@pytest.mark.parametrize("B,I,O,deg", [
    (256, 64, 64, 8), (7, 3, 5, 1), (65, 31, 33, 2), (300, 40, 70, 3), (33, 100, 100, 5),
    (200, 72, 50, 15), (129, 64, 96, 16), (64, 33, 17, 0), (1, 512, 96, 8),
])
def test_fp64_forward_backward_parity(B, I, O, deg):
    from kan_amd import functional as F
    print(f"fp64 parity B={B} I={I} O={O} deg={deg}", flush=True)
    g = torch.Generator().manual_seed(B * 3 + I + deg)
    x = torch.randn(B, I, generator=g, dtype=torch.float64) * 1.5
    c = torch.randn(I, O, deg + 1, generator=g, dtype=torch.float64) / (I * (deg + 1))
    dy = torch.randn(B, O, generator=g, dtype=torch.float64)
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c, dy)
    xd = x.cuda().requires_grad_(True)
    cd = c.cuda().requires_grad_(True)
    y = F.chebykan(xd, cd)
    assert y.dtype == torch.float64
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    assert _rel(y, y_ref) <= FP64_TOL
    assert _rel(xd.grad, dx_ref) <= FP64_TOL
    assert _rel(cd.grad, dc_ref) <= FP64_TOL


def test_fp64_module_double_and_accumulation():
    import kan_amd
    torch.manual_seed(3)
    layer = kan_amd.ChebyKANLayer(48, 20, 6).double()
    c_ref = layer.cheby_coeffs.detach().clone()
    layer = layer.cuda()
    x = torch.randn(70, 48, dtype=torch.float64)
    dy = torch.randn(70, 20, dtype=torch.float64)
    y = layer(x.cuda())
    y.backward(dy.cuda())
    y2 = layer(x.cuda())
    y2.backward(dy.cuda())  # accumulates into .grad
    torch.cuda.synchronize()
    y_ref, _, dc_ref = orc.layer_forward_backward(x, c_ref, dy, need_dx=False)
    assert _rel(y2, y_ref) <= FP64_TOL
    assert _rel(layer.cheby_coeffs.grad, 2 * dc_ref) <= FP64_TOL


def test_fp64_empty_batch_zeroes_grad():
    from kan_amd import _lib
    lib = _lib.load()
    I, O, deg = 5, 4, 3
    d = _lib.make_desc(0, I, O, deg, 0, 0)
    dc = torch.full((I, O, deg + 1), 7.0, dtype=torch.float64, device="cuda")
    st = _lib.stream_ptr(dc.device)
    _lib.check(lib.ckan_backward_f64(d, None, None, None, None, dc.data_ptr(), 0, st))
    torch.cuda.synchronize()
    assert torch.count_nonzero(dc).item() == 0
    bad = _lib.make_desc(4, I, O, deg, 1, 0)  # bf16 compute makes no sense for fp64
    assert lib.ckan_forward_f64(bad, 16, 16, 16, 16, st) == _lib.CKAN_ERR_INVALID_ARG


@pytest.mark.parametrize("family,deg,alpha,beta", [
    ("jacobi", 8, 0.5, 0.5), ("jacobi", 12, -0.3, 1.2), ("jacobi", 20, 0.0, 0.0),
    ("hermite", 8, 0.0, 0.0), ("hermite", 12, 0.0, 0.0), ("hermite_e", 10, 0.0, 0.0),
])
def test_fp64_family_layers_match_oracle(family, deg, alpha, beta):
    """JacobiKANLayer / HermiteKANLayer after .double(): the reference computes
    their bases in fp64 (kan/basis/jacobi.py:96-117, kan/basis/hermite.py:118-139).
    y, dx and dC against the oracle's op-for-op restatement run in fp64 (the
    reference's recurrences), and against the closed forms (power sums, whose
    cancellation at these degrees costs a few more bits: 1e-10)."""
    import kan_amd
    from oracle import family_oracle as fo
    print(f"fp64 family {family} deg={deg}", flush=True)
    torch.manual_seed(11 + deg)
    I, O, B = 40, 24, 90
    if family == "jacobi":
        layer = kan_amd.JacobiKANLayer(I, O, deg, alpha=alpha, beta=beta)
    else:
        layer = kan_amd.HermiteKANLayer(I, O, deg, scaling="physicist" if family == "hermite"
                                        else "probabilist")
    layer = layer.double()
    c = layer.get_coefficients().detach().clone()
    layer = layer.cuda()
    g = torch.Generator().manual_seed(deg)
    x = torch.randn(B, I, generator=g, dtype=torch.float64)
    dy = torch.randn(B, O, generator=g, dtype=torch.float64)
    xd = x.cuda().requires_grad_(True)
    y = layer(xd)
    assert y.dtype == torch.float64
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    dc = layer.get_coefficients().grad
    y_ref, dx_ref, dc_ref = fo.family_forward_backward(x, c, dy, family, alpha, beta)
    assert _rel(y, y_ref) <= FP64_TOL
    assert _rel(xd.grad, dx_ref) <= FP64_TOL
    assert _rel(dc, dc_ref) <= FP64_TOL
    y_cf = fo.family_forward_fp64(x.numpy(), c.numpy(), family, alpha, beta)
    dx_cf, dc_cf = fo.family_backward_fp64(x.numpy(), c.numpy(), dy.numpy(), family, alpha, beta)
    assert _rel(y, torch.from_numpy(y_cf)) <= 1e-10
    assert _rel(xd.grad, torch.from_numpy(dx_cf)) <= 1e-10
    assert _rel(dc, torch.from_numpy(dc_cf)) <= 1e-10


def test_fp64_finite_domain_hermite_raises():
    """The affine input map of a finite-domain Hermite layer carries its scale
    and shift in fp32 (ckan_desc), so the fp64 path refuses it clearly."""
    import kan_amd
    layer = kan_amd.HermiteKANLayer(6, 4, 5, domain=(-2.0, 3.0)).double().cuda()
    with pytest.raises(RuntimeError, match="finite domain"):
        layer(torch.randn(3, 6, dtype=torch.float64).cuda())
