"""GPU parity of ChebyKAN layers above degree 16 (the reference layer takes
any degree: kan/layers/chebykan.py:21-51, kan/basis/chebyshev.py:78-101).

Those layers run on the vector-ALU kernels in fp32, the degree axis in
chunks of 17 (the cases below cover one chunk and a remainder of 1, whole
chunks, several chunks with a short last one, degree 256, and up to 1024, the largest served).  The oracle runs in fp64 here: the fp32 acos/cos of the reference's
default path itself drifts by about d * 6e-8 at degree d, so the fp64 form is
the honest yardstick.

Tolerances (norm-wise, ||a - b|| / ||b||):
  fp32:  1e-5 for y, dx and dC (an fp32 recurrence against the exact fp64
         value stays below 6e-6 up to degree 256 on these inputs); above
         256, 1.2e-7 per degree (the recurrence's rounding grows linearly
         with the degree: 1.2e-4 at 1024)
  fp64:  1e-11
A bf16 compute request runs the same fp32 kernels (asserted bit-identical);
bf16 coefficients are widened to fp32 and compared against the oracle on the
same bf16-rounded values.
"""

import pytest
import torch

from oracle import chebykan_oracle as orc

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
FP64_TOL = 1e-11


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    n = b.norm().item()
    return (a - b).norm().item() / (n if n > 0 else 1.0)


def _inputs(B, I, O, deg, seed, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, I, generator=g, dtype=torch.float64) * 1.5).to(dtype)
    c = (torch.randn(I, O, deg + 1, generator=g, dtype=torch.float64) / (I * (deg + 1))).to(dtype)
    dy = torch.randn(B, O, generator=g, dtype=torch.float64).to(dtype)
    return x, c, dy


def _gpu(x, c, dy, compute="fp32"):
    from kan_amd import functional as F
    xd = x.cuda().requires_grad_(True)
    cd = c.cuda().requires_grad_(True)
    y = F.chebykan(xd, cd, compute)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    return y.detach().cpu(), xd.grad.cpu(), cd.grad.cpu()


@pytest.mark.parametrize("B,I,O,deg", [
    (64, 8, 8, 17),       # one chunk of 17 and one of 1
    (200, 33, 20, 24),
    (129, 16, 50, 33),    # two full chunks
    (70, 9, 13, 35),      # three chunks, the last of 2 degrees
    (33, 5, 7, 64),
    (300, 70, 130, 20),   # several output and input tiles, ragged
    (16, 4, 3, 256),
    (24, 5, 4, 600),      # 36 chunks, the last of 6 degrees
    (16, 3, 3, 1024),     # the largest degree served (12 KiB recurrence block in LDS)
    (1, 3, 2, 40),
])
def test_high_degree_fp32_parity(B, I, O, deg):
    print(f"high degree fp32 B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=B + 7 * deg)
    y, dx, dc = _gpu(x, c, dy)
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x.double(), c.double(), dy.double())
    tol = max(FP32_TOL, 1.2e-7 * deg)
    assert _rel(y, y_ref) <= tol
    assert _rel(dx, dx_ref) <= tol
    assert _rel(dc, dc_ref) <= tol


def test_high_degree_bf16_request_runs_fp32():
    print("high degree bf16 request", flush=True)
    x, c, dy = _inputs(150, 24, 40, 20, seed=11)
    a = _gpu(x, c, dy, "fp32")
    b = _gpu(x, c, dy, "bf16")
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_high_degree_bf16_coefficients():
    print("high degree bf16 coefficients", flush=True)
    x, c, dy = _inputs(96, 12, 18, 30, seed=12)
    cb = c.to(torch.bfloat16)
    y, dx, dc = _gpu(x, cb, dy)
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x.double(), cb.double(), dy.double())
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(dx, dx_ref) <= FP32_TOL
    assert _rel(dc.float(), dc_ref) <= 1e-2  # dC is returned in the coefficients' dtype (bf16)


@pytest.mark.parametrize("B,I,O,deg", [(90, 20, 30, 40), (17, 5, 6, 17), (40, 8, 9, 100), (9, 3, 4, 1024)])
def test_high_degree_fp64_parity(B, I, O, deg):
    print(f"high degree fp64 B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=3 * B + deg, dtype=torch.float64)
    y, dx, dc = _gpu(x, c, dy)
    assert y.dtype == torch.float64
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c, dy)
    assert _rel(y, y_ref) <= FP64_TOL
    assert _rel(dx, dx_ref) <= FP64_TOL
    assert _rel(dc, dc_ref) <= FP64_TOL


def test_high_degree_module_accumulates_grad():
    import kan_amd
    print("high degree module", flush=True)
    torch.manual_seed(5)
    layer = kan_amd.ChebyKANLayer(24, 10, 21)
    c_ref = layer.cheby_coeffs.detach().clone()
    layer = layer.cuda()
    g = torch.Generator().manual_seed(6)
    x = torch.randn(4, 5, 24, generator=g)  # flattened to [-1, in] like the reference
    dy = torch.randn(20, 10, generator=g)
    for _ in range(2):
        y = layer(x.cuda())
        y.backward(dy.cuda())  # the layer returns [-1, out] (chebykan.py:53-67)
    torch.cuda.synchronize()
    y_ref, _, dc_ref = orc.layer_forward_backward(x.view(-1, 24).double(), c_ref.double(),
                                                  dy.double(), need_dx=False)
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(layer.cheby_coeffs.grad, 2 * dc_ref) <= FP32_TOL


def test_high_degree_empty_batch_and_noalloc():
    from kan_amd import _lib
    print("high degree empty batch / noalloc", flush=True)
    lib = _lib.load()
    I, O, deg, B = 6, 5, 19, 33
    st = _lib.stream_ptr(torch.device("cuda"))
    d0 = _lib.make_desc(0, I, O, deg, 0, 0)
    dc = torch.full((I, O, deg + 1), 7.0, device="cuda")
    _lib.check(lib.ckan_backward(d0, None, None, None, None, dc.data_ptr(), 0, None, 0, st))
    torch.cuda.synchronize()
    assert torch.count_nonzero(dc).item() == 0
    d = _lib.make_desc(B, I, O, deg, 0, 0)
    assert lib.ckan_fwd_workspace_bytes(d) == 0
    x, c, _ = _inputs(B, I, O, deg, seed=9)
    xd, cd = x.cuda(), c.cuda()
    packed = torch.empty(lib.ckan_packed_bytes(d), dtype=torch.uint8, device="cuda")
    _lib.check(lib.ckan_pack_coeffs(d, cd.data_ptr(), packed.data_ptr(), st))
    outs = []
    for fn in ("forward", "noalloc"):
        t = torch.empty(lib.ckan_tcache_elems(d), device="cuda")
        y = torch.empty(B, O, device="cuda")
        if fn == "forward":
            _lib.check(lib.ckan_forward(d, xd.data_ptr(), packed.data_ptr(), y.data_ptr(),
                                        t.data_ptr(), None, 0, st))
        else:
            _lib.check(lib.ckan_forward_noalloc(d, xd.data_ptr(), packed.data_ptr(), y.data_ptr(),
                                                t.data_ptr(), st))
        torch.cuda.synchronize()
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1])
    y_ref = orc.layer_forward(x.double(), c.double())
    assert _rel(outs[0], y_ref) <= FP32_TOL


@pytest.mark.parametrize("optimizer", ["sgd", "adam"])
def test_high_degree_executor_matches_oracle(optimizer):
    from kan_amd import ResidentExecutor
    print(f"high degree executor {optimizer}", flush=True)
    widths, degrees, B = [20, 24, 6], [24, 18], 96
    g = torch.Generator().manual_seed(14)
    x = torch.rand(B, 20, generator=g) * 4 - 2
    y = torch.sin(x[:, :6]) + 0.05 * torch.randn(B, 6, generator=g)
    torch.manual_seed(15)
    coeffs = [orc.init_coeffs(widths[l], widths[l + 1], degrees[l]) for l in range(2)]
    lr = 0.05 if optimizer == "sgd" else 1e-3
    ex = ResidentExecutor(widths, degrees, B, compute="fp32", loss="mse", optimizer=optimizer,
                          lr=lr, weight_decay=0.01)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    losses = [ex.step(x.cuda(), y.cuda()).item() for _ in range(3)]
    c_ref, losses_ref = orc.train_steps(x.double(), y.double(), [c.double() for c in coeffs],
                                        steps=3, loss="mse", optimizer=optimizer, lr=lr,
                                        weight_decay=0.01)
    for a, b in zip(losses, losses_ref):
        assert abs(a - b) <= 1e-5 * abs(b) + 1e-7
    for l in range(2):
        assert _rel(ex.get_coeffs(l), c_ref[l]) <= 1e-5
    ex.close()


# Jacobi / Hermite layers above degree 16: the vector-ALU kernels run the
# family's own three-term recurrence (coefficients from the packed buffer's
# recurrence block) and differentiate it for dx, so dC comes out in the
# family's basis directly.  Oracle: the reference's op order
# (oracle/family_oracle.py) evaluated in fp64; the same op order in fp32
# stays within 5.1e-6 of it on these cases (Jacobi(1.5, 0.5) at degree 40 the
# largest).
FAMILY_CASES = [
    # family, alpha, beta, B, I, O, deg
    ("jacobi", 0.0, 0.0, 200, 33, 20, 24),
    ("jacobi", 1.5, 0.5, 129, 16, 50, 40),   # three chunks
    ("jacobi", -0.5, 0.25, 64, 8, 8, 17),    # a chunk of 17 and one of 1
    ("jacobi", 0.5, 0.5, 16, 4, 3, 100),
    ("jacobi", 0.5, 0.5, 12, 3, 4, 500),     # the recurrence block of 501 degrees in LDS
    ("hermite", 0, 0, 70, 9, 13, 20),
    ("hermite", 0, 0, 40, 6, 5, 32),
    ("hermite_e", 0, 0, 150, 24, 40, 30),
]


def _family_spec(family, deg, alpha=0.0, beta=0.0):
    from kan_amd import _lib
    if family == "jacobi":
        return _lib.make_spec(_lib.CKAN_BASIS_JACOBI, deg, alpha, beta, 1.0)
    fam = _lib.CKAN_BASIS_HERMITE if family == "hermite" else _lib.CKAN_BASIS_HERMITE_E
    return _lib.make_spec(fam, deg, 0.0, 0.0, 3.0)


def _family_gpu(x, c, dy, spec, compute="fp32", affine=None):
    from kan_amd import functional as F
    xd = x.cuda().requires_grad_(True)
    cd = c.cuda().requires_grad_(True)
    y = F.family_kan(xd, cd, spec, compute, affine)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    return y.detach().cpu(), xd.grad.cpu(), cd.grad.cpu()


@pytest.mark.parametrize("family,alpha,beta,B,I,O,deg", FAMILY_CASES)
def test_high_degree_family_parity(family, alpha, beta, B, I, O, deg):
    from oracle import family_oracle as fo
    print(f"high degree {family}({alpha},{beta}) B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=B + deg)
    y, dx, dc = _family_gpu(x, c, dy, _family_spec(family, deg, alpha, beta))
    y_ref, dx_ref, dc_ref = fo.family_forward_backward(x.double(), c.double(), dy.double(),
                                                       family, alpha, beta)
    tol = max(FP32_TOL, 1.2e-7 * deg)
    assert _rel(y, y_ref) <= tol
    assert _rel(dx, dx_ref) <= tol
    assert _rel(dc, dc_ref) <= tol


def test_high_degree_family_bf16_request_runs_fp32():
    print("high degree family bf16 request", flush=True)
    x, c, dy = _inputs(90, 12, 20, 22, seed=21)
    spec = _family_spec("jacobi", 22, 0.5, -0.5)
    a = _family_gpu(x, c, dy, spec, "fp32")
    b = _family_gpu(x, c, dy, spec, "bf16")
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.parametrize("scaling,B,I,O,deg", [("physicist", 120, 20, 30, 20),
                                                ("probabilist", 33, 7, 9, 28)])
def test_high_degree_hermite_finite_domain(scaling, B, I, O, deg):
    """HermiteKANLayer(domain=(lo, hi), normalize_domain=True) above degree
    16: the affine map onto [-3, 3] (kan/basis/hermite.py:102-112) runs in the
    vector-ALU input-map launch, dx takes its constant chain factor; the
    coefficient gradient accumulates over two backward calls."""
    import kan_amd
    from oracle import family_oracle as fo
    print(f"high degree hermite affine {scaling} B={B} I={I} O={O} deg={deg}", flush=True)
    dom = (-2.0, 5.0)
    torch.manual_seed(B + deg)
    m = kan_amd.HermiteKANLayer(I, O, deg, scaling=scaling, domain=dom, normalize_domain=True)
    c = m.hermite_coeffs.detach().clone()
    g = torch.Generator().manual_seed(B + I)
    x = torch.rand(B, I, generator=g) * 7.6 - 2.3  # partly outside [lo, hi]
    dy = torch.randn(B, O, generator=g)
    fam = "hermite" if scaling == "physicist" else "hermite_e"
    y_ref, dx_ref, dc_ref = fo.family_forward_backward(x.double(), c.double(), dy.double(), fam,
                                                       domain=dom)
    m = m.cuda()
    for _ in range(2):
        xd = x.cuda().requires_grad_(True)
        y = m(xd)
        y.backward(dy.cuda())
    torch.cuda.synchronize()
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(xd.grad, dx_ref) <= FP32_TOL
    assert _rel(m.hermite_coeffs.grad, 2 * dc_ref) <= FP32_TOL


def test_high_degree_family_coeff_grad_map_is_identity():
    """ckan_coeff_grad_from_chebyshev above degree 16 (where the backward
    already differentiates in the family's basis): a copy, an accumulation,
    and nothing in place."""
    from kan_amd import _lib
    print("high degree family coefficient-gradient map", flush=True)
    lib = _lib.load()
    I, O, deg = 9, 11, 30
    spec = _family_spec("hermite_e", deg)
    d = _lib.make_desc(4, I, O, deg, 0, 0)
    st = _lib.stream_ptr(torch.device("cuda"))
    g = torch.Generator().manual_seed(31)
    src = torch.randn(I, O, deg + 1, generator=g).cuda()
    base = torch.randn(I, O, deg + 1, generator=g).cuda()
    out = torch.empty_like(src)
    _lib.check(lib.ckan_coeff_grad_from_chebyshev(d, spec, src.data_ptr(), out.data_ptr(), 0, st))
    acc = base.clone()
    _lib.check(lib.ckan_coeff_grad_from_chebyshev(d, spec, src.data_ptr(), acc.data_ptr(), 1, st))
    same = src.clone()
    _lib.check(lib.ckan_coeff_grad_from_chebyshev(d, spec, same.data_ptr(), same.data_ptr(), 0, st))
    torch.cuda.synchronize()
    assert torch.equal(out, src)
    assert torch.equal(acc, base + src)
    assert torch.equal(same, src)


@pytest.mark.parametrize("family,alpha,beta,deg", [("jacobi", 1.0, 0.5, 40), ("hermite", 0, 0, 24),
                                                   ("hermite_e", 0, 0, 40)])
def test_high_degree_family_basis_functions(family, alpha, beta, deg):
    """The materialised family basis and its backward above degree 16
    (kan/basis/jacobi.py:119-188, kan/basis/hermite.py:141-233), against the
    reference's recurrence in fp64."""
    from kan_amd import functional as F
    from oracle import family_oracle as fo
    print(f"high degree {family} basis deg={deg}", flush=True)
    s = 1.0 if family == "jacobi" else 3.0
    t = (torch.rand(300, 7, generator=torch.Generator().manual_seed(1)) * 2 - 1) * s
    g = torch.randn(300, 7, deg + 1, generator=torch.Generator().manual_seed(2))
    tr = t.clone().double().requires_grad_(True)
    ref = fo.family_basis(tr, family, deg, alpha, beta)
    (ref * g.double()).sum().backward()
    td = t.cuda().requires_grad_(True)
    out = F.family_basis(td, _family_spec(family, deg, alpha, beta))
    (out * g.cuda()).sum().backward()
    torch.cuda.synchronize()
    assert _rel(out, ref) <= FP32_TOL
    assert _rel(td.grad, tr.grad) <= FP32_TOL
