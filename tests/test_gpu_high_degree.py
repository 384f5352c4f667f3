"""GPU parity of ChebyKAN layers above degree 16 (the reference layer takes
any degree: kan/layers/chebykan.py:21-51, kan/basis/chebyshev.py:78-101).

Those layers run on the vector-ALU kernels in fp32, the degree axis in
chunks of 17 (several launches, each advancing the recurrence to its first
degree).  The oracle runs in fp64 here: the fp32 acos/cos of the reference's
default path itself drifts by about d * 6e-8 at degree d, so the fp64 form is
the honest yardstick.

Tolerances (norm-wise, ||a - b|| / ||b||):
  fp32:  1e-5 for y, dx and dC (an fp32 recurrence against the exact fp64
         value stays below 6e-6 up to degree 256 on these inputs)
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
    (16, 4, 3, 256),      # the largest degree served
    (1, 3, 2, 40),
])
def test_high_degree_fp32_parity(B, I, O, deg):
    print(f"high degree fp32 B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=B + 7 * deg)
    y, dx, dc = _gpu(x, c, dy)
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x.double(), c.double(), dy.double())
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(dx, dx_ref) <= FP32_TOL
    assert _rel(dc, dc_ref) <= FP32_TOL


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


@pytest.mark.parametrize("B,I,O,deg", [(90, 20, 30, 40), (17, 5, 6, 17), (40, 8, 9, 100)])
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
