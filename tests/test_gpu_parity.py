"""GPU parity: the HIP path (through the C-ABI) against the CPU oracle.

Tolerances (norm-wise, ||a - b|| / ||b||):
  fp32 MFMA path:  1e-5 for y, dx and dC
  bf16 MFMA path:  2e-2, against the fp32 oracle applied to the same
                   bf16-rounded coefficients (the reference cannot run bf16
                   coefficients itself)
Inputs keep |x| < 9 so the reference's saturation NaN (|x| >= 9.0108) does
not arise; that divergence is tested separately.
"""
import io
import math

import numpy as np
import pytest
import torch

from oracle import chebykan_oracle as orc

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 2e-2


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    n = b.norm().item()
    return (a - b).norm().item() / (n if n > 0 else 1.0)


def _inputs(B, I, O, deg, seed, x_scale=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, I, generator=g) * x_scale
    c = torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))
    dy = torch.randn(B, O, generator=g)
    return x, c, dy


def _gpu_fwd_bwd(x, c, dy, compute, need_dx=True, need_dc=True):
    from kan_amd import functional as F
    xd = x.cuda().requires_grad_(need_dx)
    cd = c.cuda().requires_grad_(need_dc)
    y = F.chebykan(xd, cd, compute)
    y.backward(dy.cuda())
    torch.cuda.synchronize()
    return (y.detach().cpu(), xd.grad.cpu() if need_dx else None,
            cd.grad.cpu() if need_dc else None)


SHAPES = [
    # B, I, O, deg
    (100, 1, 1, 8),       # config 1
    (256, 784, 64, 4),    # config 2 layer 1
    (256, 64, 10, 4),     # config 2 layer 2
    (64, 33, 17, 0),
    (7, 3, 5, 1),
    (65, 31, 33, 2),
    (300, 40, 70, 3),
    (33, 100, 100, 5),
    (129, 64, 96, 7),
    (512, 256, 256, 8),
    (96, 48, 40, 9),
    (200, 72, 50, 15),
    (256, 128, 64, 16),
    (1000, 100, 150, 6),  # pipelined forward: ragged rows, padded inputs, partial tiles
    (777, 40, 300, 12),   # the same at degree 16 (P = 16)
    (50, 100, 70, 6),     # streaming forward, 33..64 rows (tanh from the cache), padded inputs
    (300, 50, 130, 16),   # degree-16 dx on 16-input blocks: ragged rows, inputs and outputs
    (520, 272, 96, 13),   # the same past one 256-row block, 17 input blocks
    (4096, 600, 64, 16),  # degree-16 dx, 608 tiles over 256 persistent blocks, 2 stages each
    (2048, 1040, 512, 15),  # the same with 16 stages per tile, 65 input blocks
    (5, 40, 100, 16),     # degree-16 dx with 5 rows: one partial tile per input block
    (2100, 1000, 136, 7),  # bf16 dx with copy waves: 288 tiles over 256 persistent blocks
                           # (two tiles for some), ragged rows / inputs / outputs, 6 stages
    (2600, 900, 130, 4),   # the same at degree 4: 319 tiles, 4 stages per tile
    (1500, 200, 40, 8),    # pipelined forward, 64-column tile (<= 64 outputs): ragged second fragment
    (1024, 96, 20, 3),     # the same with one output fragment, degree 3
    (3000, 130, 64, 12),   # the same at degree 16 (P = 16), ragged rows and inputs
]


@pytest.mark.parametrize("B,I,O,deg", SHAPES)
def test_fp32_forward_backward_parity(B, I, O, deg):
    print(f"fp32 parity B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=B * 7 + I + deg, x_scale=1.5)
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c, dy)
    y, dx, dc = _gpu_fwd_bwd(x, c, dy, "fp32")
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(dx, dx_ref) <= FP32_TOL
    assert _rel(dc, dc_ref) <= FP32_TOL


@pytest.mark.parametrize("B,I,O,deg", SHAPES)
def test_bf16_forward_backward_parity(B, I, O, deg):
    print(f"bf16 parity B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=B * 5 + O + deg, x_scale=1.5)
    c_r = c.bfloat16().float()
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c_r, dy)
    y, dx, dc = _gpu_fwd_bwd(x, c_r, dy, "bf16")
    assert _rel(y, y_ref) <= BF16_TOL
    assert _rel(dx, dx_ref) <= BF16_TOL
    assert _rel(dc, dc_ref) <= BF16_TOL


def test_fp32_config3_scaled_parity():
    # config 3 shape with the batch cut to 1024 rows so the CPU oracle is quick
    print("fp32 parity cfg3 B=1024", flush=True)
    x, c, dy = _inputs(1024, 1024, 1024, 8, seed=3)
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c, dy)
    y, dx, dc = _gpu_fwd_bwd(x, c, dy, "fp32")
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(dx, dx_ref) <= FP32_TOL
    assert _rel(dc, dc_ref) <= FP32_TOL


@pytest.mark.parametrize("compute,tol", [("fp32", FP32_TOL), ("bf16", BF16_TOL)])
def test_config3_full_size_unrounded_parity(compute, tol):
    """Full config 3 (B=8192, 1024->1024, deg 8) on fp32 coefficients that are
    not bf16 values, every row: y, dx and dC against the oracle.  For bf16
    the oracle takes C rounded to bf16, so the pack's own fp32 -> bf16
    rounding is what is pinned at this size (the oracle's full step takes
    about half a second on 16 host cores)."""
    print(f"cfg3 full-size unrounded parity {compute}", flush=True)
    x, c, dy = _inputs(8192, 1024, 1024, 8, seed=41, x_scale=1.5)
    assert not torch.equal(c, c.bfloat16().float())
    y, dx, dc = _gpu_fwd_bwd(x, c, dy, compute)
    c_ref = c.bfloat16().float() if compute == "bf16" else c
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c_ref, dy)
    assert _rel(y, y_ref) <= tol
    assert _rel(dx, dx_ref) <= tol
    assert _rel(dc, dc_ref) <= tol
    if compute == "bf16":
        # the forward operand (the first region of the packed buffer: 32
        # column fragments x 512 k-blocks x 512 bf16 at this shape) holds
        # C[i, o, d >= 1] rounded to bf16: the same bytes whether the pack
        # rounds C itself or C arrives rounded by torch (round to nearest even)
        import ctypes
        from kan_amd import _lib
        lib = _lib.load()
        d = _lib.make_desc(8192, 1024, 1024, 8, _lib.CKAN_COMPUTE_BF16, _lib.CKAN_DTYPE_F32)
        s = _lib.stream_ptr(torch.device("cuda"))
        nb = lib.ckan_packed_bytes(ctypes.byref(d))
        cf_bytes = 32 * 512 * 512 * 2
        packs = []
        for cc in (c, c_ref):
            pk = torch.zeros(nb, dtype=torch.uint8, device="cuda")
            cd = cc.cuda()
            _lib.check(lib.ckan_pack_coeffs(ctypes.byref(d), cd.data_ptr(), pk.data_ptr(), s))
            packs.append(pk)
        torch.cuda.synchronize()
        assert torch.equal(packs[0][:cf_bytes], packs[1][:cf_bytes])
        assert not torch.equal(packs[0][cf_bytes:], packs[1][cf_bytes:])  # dX operand and fp32 bias differ


@pytest.mark.parametrize("compute,tol", [("fp32", FP32_TOL), ("bf16", BF16_TOL)])
def test_config3_full_size_properties(compute, tol):
    """Full config 3 (B=8192, 1024->1024, deg 8): row-local parity on sampled
    rows, and the size-independent identity <dC, C> = <dy, y>."""
    print(f"cfg3 full-size properties {compute}", flush=True)
    B, I, O, deg = 8192, 1024, 1024, 8
    g = torch.Generator().manual_seed(33)
    x = torch.randn(B, I, generator=g)
    c = torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))
    if compute == "bf16":
        c = c.bfloat16().float()
    dy = torch.randn(B, O, generator=g)
    y, dx, dc = _gpu_fwd_bwd(x, c, dy, compute)
    rows = torch.arange(0, B, 97)
    y_ref, dx_ref, _ = orc.layer_forward_backward(x[rows], c, dy[rows], need_dc=False)
    assert _rel(y[rows], y_ref) <= tol
    assert _rel(dx[rows], dx_ref) <= tol
    lhs = (dc.double() * c.double()).sum().item()
    rhs = (dy.double() * y.double()).sum().item()
    scale = (dc.double().abs() * c.double().abs()).sum().item()
    assert abs(lhs - rhs) <= tol * scale
    # dC columns for a few inputs, from the fp64 definition
    t = torch.tanh(x.double())
    for i in (0, 511, 1023):
        basis = torch.from_numpy(orc.cheb_T_fp64(t[:, i].numpy(), deg))  # [B, D]
        ref = basis.T @ dy.double()                                      # [D, O]
        assert _rel(dc[i].T, ref) <= tol


@pytest.mark.parametrize("B", [1, 16, 64])
def test_config5_small_batch_bf16_coeffs(B):
    """Config 5: 2048 -> 2048, deg 8, bf16 coefficients, B in {1, 16, 64}."""
    print(f"cfg5 small batch B={B}", flush=True)
    from kan_amd import functional as F
    I = O = 2048
    deg = 8
    g = torch.Generator().manual_seed(50 + B)
    x = torch.randn(B, I, generator=g)
    c = (torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))).bfloat16()
    y = F.chebykan(x.cuda(), c.cuda(), "bf16")
    torch.cuda.synchronize()
    y_ref = orc.layer_forward(x, c.float())
    assert _rel(y.cpu(), y_ref) <= BF16_TOL
    # repeated calls give bitwise the same result
    y2 = F.chebykan(x.cuda(), c.cuda(), "bf16")
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), y2.cpu())


@pytest.mark.parametrize("B,I,O,deg", [
    (1, 1000, 2048, 8),    # ragged reduction (the last wave's range is partial)
    (3, 256, 2050, 8),     # ragged columns: the last block has 2 of its columns
    (2, 300, 2048, 4),     # degree 4 (two inputs per basis vector)
    (2, 200, 2080, 2),     # degree 2 (four inputs per basis vector)
    (3, 200, 2048, 2),     # degree 2 past 2 rows: the split-K streaming forward
    (4, 130, 2048, 16),    # degree 16 (vectors take degree halves), 4 rows
    (3, 8, 2048, 8),       # one super-group: the rest of the batch is masked
    (4, 2048, 4096, 8),
    (5, 300, 2048, 4),     # 5..8 rows: the column-owning forward still computes tanh itself
    (8, 1000, 2048, 8),
    (7, 130, 2048, 16),    # degree 16 at 8 padded rows
    (13, 130, 2050, 16),   # 9..16 rows (reading the tanh cache): ragged rows and columns at degree 16
    (16, 2048, 2048, 8),   # config 5 at batch 16
    (17, 300, 2048, 8),    # past 16 rows: the split-K streaming forward
    (64, 130, 2048, 16),
])
def test_small_batch_wide_forward(B, I, O, deg):
    """Small batches at 2048 or more outputs (bf16), where up to 16 rows take
    the one-launch column-owning forward (up to 8 computing tanh themselves and
    writing the tanh cache, 9..16 reading the cache): y against the oracle, and
    dx / dC through the tanh cache, at shapes that exercise ragged edges."""
    print(f"small-batch wide forward B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=7 * B + I + deg)
    c = c.bfloat16().float()
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c, dy)
    y, dx, dc = _gpu_fwd_bwd(x, c, dy, "bf16")
    assert _rel(y, y_ref) <= BF16_TOL
    assert _rel(dx, dx_ref) <= BF16_TOL
    assert _rel(dc, dc_ref) <= BF16_TOL


def test_split_k_paths_fp32():
    # small batches with a long reduction select split-K in the forward and dC
    for B, I, O, deg in [(1, 512, 96, 8), (20, 300, 64, 4), (48, 1024, 32, 16)]:
        print(f"split-K B={B} I={I} O={O} deg={deg}", flush=True)
        x, c, dy = _inputs(B, I, O, deg, seed=B + I)
        y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c, dy)
        y, dx, dc = _gpu_fwd_bwd(x, c, dy, "fp32")
        assert _rel(y, y_ref) <= FP32_TOL
        assert _rel(dx, dx_ref) <= FP32_TOL
        assert _rel(dc, dc_ref) <= FP32_TOL


@pytest.mark.parametrize("B,I,O,deg,compute", [
    (128, 1024, 1024, 8, "bf16"),   # pipelined dC, one split: accumulates in its epilogue
    (1024, 100, 70, 5, "bf16"),     # pipelined dC, split batch: accumulates in the split sum
    (64, 48, 40, 15, "fp32"),       # fp32 degree 16: older dC kernel + finalize
])
def test_backward_accumulate_into_existing_grad(B, I, O, deg, compute):
    """ckan_backward(accumulate=1) adds to dcoeffs: R + G elementwise, bit for bit."""
    from kan_amd import _lib
    print(f"accumulate B={B} I={I} O={O} deg={deg} {compute}", flush=True)
    L = _lib.load()
    x, c, dy = _inputs(B, I, O, deg, seed=B + deg)
    code = _lib.CKAN_COMPUTE_BF16 if compute == "bf16" else _lib.CKAN_COMPUTE_FP32
    d = _lib.make_desc(B, I, O, deg, code, _lib.CKAN_DTYPE_F32)
    st = torch.cuda.current_stream().cuda_stream
    xd, cd, dyd = x.cuda(), c.cuda(), dy.cuda()
    packed = torch.empty(L.ckan_packed_bytes(d), dtype=torch.uint8, device="cuda")
    t = torch.empty(L.ckan_tcache_elems(d), device="cuda")
    y = torch.empty(B, O, device="cuda")
    fwb = max(L.ckan_fwd_workspace_bytes(d), 256)
    fws = torch.empty(fwb, dtype=torch.uint8, device="cuda")
    bwb = L.ckan_bwd_workspace_bytes(d, 0, 1)
    bws = torch.empty(bwb, dtype=torch.uint8, device="cuda")
    _lib.check(L.ckan_pack_coeffs(d, cd.data_ptr(), packed.data_ptr(), st))
    _lib.check(L.ckan_forward(d, xd.data_ptr(), packed.data_ptr(), y.data_ptr(), t.data_ptr(),
                              fws.data_ptr(), fwb, st))
    g = torch.empty(I, O, deg + 1, device="cuda")
    _lib.check(L.ckan_backward(d, t.data_ptr(), packed.data_ptr(), dyd.data_ptr(), None,
                               g.data_ptr(), 0, bws.data_ptr(), bwb, st))
    r = torch.randn(I, O, deg + 1, generator=torch.Generator().manual_seed(7)).cuda()
    acc = r.clone()
    _lib.check(L.ckan_backward(d, t.data_ptr(), packed.data_ptr(), dyd.data_ptr(), None,
                               acc.data_ptr(), 1, bws.data_ptr(), bwb, st))
    torch.cuda.synchronize()
    assert torch.equal(acc, r + g)
    _, _, dc_ref = orc.layer_forward_backward(x, c, dy, need_dx=False)
    tol = BF16_TOL if compute == "bf16" else FP32_TOL
    assert _rel(g, dc_ref) <= tol


def test_integration_ctypes_stub():
    """The minimal ctypes binding a maintainer of the reference would add
    (the stub printed in the integration notes), run as written."""
    import ctypes
    from kan_amd import _lib
    _L = ctypes.CDLL(_lib.LIB_PATH)
    for _f in ("ckan_packed_bytes", "ckan_tcache_elems", "ckan_fwd_workspace_bytes"):
        getattr(_L, _f).restype = ctypes.c_size_t
    _vp = ctypes.c_void_p

    class _Desc(ctypes.Structure):
        _fields_ = [("batch", ctypes.c_int64), ("in_dim", ctypes.c_int32), ("out_dim", ctypes.c_int32),
                    ("degree", ctypes.c_int32), ("compute", ctypes.c_int32),
                    ("coeff_dtype", ctypes.c_int32), ("input_map", ctypes.c_int32),
                    ("in_scale", ctypes.c_float), ("in_shift", ctypes.c_float)]

    def chebykan_forward(x, C):
        d = _Desc(x.shape[0], C.shape[0], C.shape[1], C.shape[2] - 1, 0, 0, 0, 0.0, 0.0)
        s = torch.cuda.current_stream().cuda_stream
        packed = torch.empty(_L.ckan_packed_bytes(ctypes.byref(d)), dtype=torch.uint8, device=x.device)
        t = torch.empty(_L.ckan_tcache_elems(ctypes.byref(d)), device=x.device)
        y = torch.empty(x.shape[0], C.shape[1], device=x.device)
        wsb = _L.ckan_fwd_workspace_bytes(ctypes.byref(d))
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=x.device)
        assert _L.ckan_pack_coeffs(ctypes.byref(d), _vp(C.data_ptr()), _vp(packed.data_ptr()), _vp(s)) == 0
        assert _L.ckan_forward(ctypes.byref(d), _vp(x.data_ptr()), _vp(packed.data_ptr()),
                               _vp(y.data_ptr()), _vp(t.data_ptr()), _vp(ws.data_ptr()),
                               ctypes.c_size_t(wsb), _vp(s)) == 0
        return y, t, packed

    for B, I, O, deg in [(300, 64, 48, 8), (8, 512, 40, 5)]:  # a tile path and a split-K path
        x, c, _ = _inputs(B, I, O, deg, seed=11)
        y, _, _ = chebykan_forward(x.cuda(), c.cuda())
        torch.cuda.synchronize()
        assert _rel(y.cpu(), orc.layer_forward(x, c)) <= FP32_TOL


def _offset_view(t):
    """A contiguous copy of t whose data pointer is 4 bytes past a 16-byte boundary."""
    full = torch.empty(t.numel() + 4, dtype=t.dtype, device=t.device)
    v = full[1:1 + t.numel()].view(t.shape)
    v.copy_(t)
    return v


@pytest.mark.parametrize("B,I,O,deg", [(512, 256, 128, 8), (16, 512, 96, 4), (300, 64, 48, 16)])
def test_misaligned_inputs_take_scalar_loads(B, I, O, deg):
    """x, dy and C at 4-byte (not 16-byte) alignment: the float4 load paths must not be taken."""
    from kan_amd import functional as F
    print(f"misaligned inputs B={B} I={I} O={O} deg={deg}", flush=True)
    x, c, dy = _inputs(B, I, O, deg, seed=B + deg)
    y_ref, dx_ref, dc_ref = orc.layer_forward_backward(x, c, dy)
    xd = _offset_view(x.cuda()).requires_grad_(True)
    cd = _offset_view(c.cuda()).requires_grad_(True)
    dyd = _offset_view(dy.cuda())
    assert xd.data_ptr() % 16 == 4 and cd.data_ptr() % 16 == 4 and dyd.data_ptr() % 16 == 4
    y = F.chebykan(xd, cd, "fp32")
    y.backward(dyd)
    torch.cuda.synchronize()
    assert _rel(y, y_ref) <= FP32_TOL
    assert _rel(xd.grad, dx_ref) <= FP32_TOL
    assert _rel(cd.grad, dc_ref) <= FP32_TOL


def test_deterministic_results():
    x, c, dy = _inputs(512, 128, 128, 8, seed=9)
    a = _gpu_fwd_bwd(x, c, dy, "bf16")
    b = _gpu_fwd_bwd(x, c, dy, "bf16")
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_only_coeff_grad_skips_dx():
    x, c, dy = _inputs(128, 64, 32, 4, seed=4)
    y_ref, _, dc_ref = orc.layer_forward_backward(x, c, dy, need_dx=False)
    y, dx, dc = _gpu_fwd_bwd(x, c, dy, "fp32", need_dx=False)
    assert dx is None
    assert _rel(dc, dc_ref) <= FP32_TOL


@pytest.mark.parametrize("compute,tol", [("fp32", FP32_TOL), ("bf16", BF16_TOL)])
def test_only_input_grad_skips_dc(compute, tol):
    x, c, dy = _inputs(512, 256, 128, 8, seed=5)
    y_ref, dx_ref, _ = orc.layer_forward_backward(x, c, dy)
    y, dx, dc = _gpu_fwd_bwd(x, c, dy, compute, need_dc=False)
    assert dc is None
    assert _rel(dx, dx_ref) <= tol


def test_saturation_is_finite_and_analytic():
    """Divergence from the reference by design: for |x| >= 9.0108 the
    reference's dx is NaN; this path returns the analytic limit."""
    x = torch.tensor([[0.0], [3.0], [9.5], [-12.0]])
    c = torch.ones(1, 1, 9)
    dy = torch.ones(4, 1)
    _, dx, _ = _gpu_fwd_bwd(x, c, dy, "fp32")
    dx64, _ = orc.backward_fp64(x.numpy(), c.numpy(), dy.numpy())
    assert torch.isfinite(dx).all()
    assert np.allclose(dx.numpy().ravel(), dx64.ravel(), rtol=1e-4, atol=1e-5)


def test_layer_module_and_state_dict_roundtrip():
    import kan_amd
    torch.manual_seed(2)
    m = kan_amd.ChebyKANLayer(16, 8, 6).cuda()
    x = torch.randn(4, 2, 16)  # forward views to [-1, in]
    y = m(x.cuda())
    assert y.shape == (8, 8)
    y_ref = orc.layer_forward(x.reshape(-1, 16), m.cheby_coeffs.detach().cpu())
    assert _rel(y.detach().cpu(), y_ref) <= FP32_TOL
    m2 = kan_amd.ChebyKANLayer(16, 8, 6).cuda()
    m2.load_state_dict(m.state_dict())
    assert torch.equal(m2(x.cuda()).detach().cpu(), y.detach().cpu())


def test_basis_functions_and_backward():
    import kan_amd
    b = kan_amd.ChebyshevBasis(degree=7)
    t = (torch.rand(50, 6) * 2 - 1)
    out = b.basis_functions(t.cuda()).cpu()
    assert _rel(out, orc.basis_closed_form(t, 7)) <= 1e-5
    td = t.cuda().requires_grad_(True)
    g = torch.randn(50, 6, 8)
    b.basis_functions(td).backward(g.cuda())
    # d/dt sum_d g_d T_d(t) = sum_d g_d d U_{d-1}(t), in fp64.  (The
    # reference's use_recurrence=True basis writes slices in place and
    # cannot be differentiated with respect to its input at all.)
    U = orc.cheb_U_fp64(t.double().numpy(), 7)
    d = np.arange(1, 8)
    ref = (g.double().numpy()[..., 1:] * d * U[..., :7]).sum(-1)
    assert _rel(td.grad.cpu(), torch.from_numpy(ref)) <= 1e-5


def test_optimizers_match_torch():
    from kan_amd import optim
    g = torch.Generator().manual_seed(8)
    p0 = torch.randn(1000, generator=g)
    grads = [torch.randn(1000, generator=g) for _ in range(5)]
    for wd in (0.0, 0.01):
        pr = p0.clone().requires_grad_(True)
        ref = torch.optim.Adam([pr], lr=0.01, weight_decay=wd)
        pd = p0.cuda().requires_grad_(True)
        opt = optim.Adam([pd], lr=0.01, weight_decay=wd)
        for gr in grads:
            pr.grad = gr.clone()
            ref.step()
            pd.grad = gr.cuda()
            opt.step()
        assert torch.allclose(pd.detach().cpu(), pr.detach(), rtol=0, atol=1e-6)
    pr = p0.clone().requires_grad_(True)
    ref = torch.optim.SGD([pr], lr=0.05)
    pd = p0.cuda().requires_grad_(True)
    opt = optim.SGD([pd], lr=0.05)
    for gr in grads:
        pr.grad = gr.clone()
        ref.step()
        pd.grad = gr.cuda()
        opt.step()
    assert torch.allclose(pd.detach().cpu(), pr.detach(), rtol=0, atol=1e-6)


def test_config1_training_loop_matches_oracle():
    """Config 1 (README.md:42-73): 1000 full-batch Adam steps on sin(2 pi x)."""
    import kan_amd
    from kan_amd import optim
    x = torch.linspace(-1, 1, 100).reshape(-1, 1)
    y = torch.sin(2 * math.pi * x)
    torch.manual_seed(0)
    m = kan_amd.ChebyKANLayer(1, 1, 8)
    c0 = m.cheby_coeffs.detach().clone()
    m = m.cuda()
    opt = optim.Adam(m.parameters(), lr=0.01)
    xd, yd = x.cuda(), y.cuda()
    losses = []
    for _ in range(1000):
        opt.zero_grad()
        loss = torch.nn.functional.mse_loss(m(xd), yd)
        loss.backward()
        opt.step()
        losses.append(loss.detach())
    losses = torch.stack(losses).cpu()
    c_ref, losses_ref = orc.train_steps(x, y, [c0], steps=1000, loss="mse", optimizer="adam", lr=0.01)
    assert abs(losses[-1].item() - losses_ref[-1]) <= 1e-3 * max(losses_ref[0], 1e-6) + 1e-5
    assert _rel(m.cheby_coeffs.detach().cpu(), c_ref[0]) <= 1e-3


@pytest.mark.parametrize("compute,tol", [("fp32", FP32_TOL), ("bf16", BF16_TOL)])
def test_use_recurrence_layer_matches_recurrence_oracle(compute, tol):
    """ChebyKANLayer(..., use_recurrence=True) (kan/basis/chebyshev.py:147-172,
    dispatch at :114-117) against the oracle's recurrence path: y and dC.  The
    reference's recurrence writes slices in place, so autograd cannot give its
    dx; dx is checked against the closed-form oracle instead."""
    import kan_amd
    B, I, O, deg = 384, 96, 80, 8
    print(f"use_recurrence layer {compute}", flush=True)
    torch.manual_seed(31)
    m = kan_amd.ChebyKANLayer(I, O, deg, use_recurrence=True, compute=compute)
    assert m.basis.use_recurrence
    c = m.cheby_coeffs.detach().clone()
    g = torch.Generator().manual_seed(32)
    x = torch.randn(B, I, generator=g) * 1.5
    dy = torch.randn(B, O, generator=g)
    c_ref = c.to(torch.bfloat16).float() if compute == "bf16" else c
    y_ref, _, dc_ref = orc.layer_forward_backward(x, c_ref, dy, need_dx=False, use_recurrence=True)
    _, dx_ref, _ = orc.layer_forward_backward(x, c_ref, dy)
    m = m.cuda()
    xd = x.cuda().requires_grad_(True)
    y = m(xd)
    y.backward(dy.cuda())
    assert _rel(y.detach().cpu(), y_ref) <= tol
    assert _rel(m.cheby_coeffs.grad.cpu(), dc_ref) <= tol
    assert _rel(xd.grad.cpu(), dx_ref) <= tol


def test_use_recurrence_at_saturation_is_exact_and_finite():
    """At |x| >= 9.0108 fp32 tanh(x) is exactly +-1, where the recurrence
    gives T_n(+-1) = (+-1)^n exactly; y and dC match the recurrence oracle and
    dx is the finite analytic limit (the reference gives no dx there)."""
    import kan_amd
    torch.manual_seed(33)
    m = kan_amd.ChebyKANLayer(3, 4, 7, use_recurrence=True)
    c = m.cheby_coeffs.detach().clone()
    x = torch.tensor([[9.5, -12.0, 0.3], [20.0, 1.0, -9.2], [0.0, -30.0, 10.0]])
    dy = torch.randn(3, 4, generator=torch.Generator().manual_seed(34))
    y_ref, _, dc_ref = orc.layer_forward_backward(x, c, dy, need_dx=False, use_recurrence=True)
    m = m.cuda()
    xd = x.cuda().requires_grad_(True)
    y = m(xd)
    y.backward(dy.cuda())
    assert _rel(y.detach().cpu(), y_ref) <= FP32_TOL
    assert _rel(m.cheby_coeffs.grad.cpu(), dc_ref) <= FP32_TOL
    dx64, _ = orc.backward_fp64(x.numpy(), c.numpy(), dy.numpy())
    assert torch.isfinite(xd.grad).all()
    assert np.allclose(xd.grad.cpu().numpy(), dx64, rtol=1e-4, atol=1e-6)


def test_adam_resumes_from_a_torch_optim_checkpoint():
    """kan_amd.optim.Adam continues a torch.optim.Adam run from its
    state_dict (step stored as a float tensor) on the device."""
    from kan_amd import optim
    g = torch.Generator().manual_seed(35)
    p0 = torch.randn(500, generator=g)
    grads = [torch.randn(500, generator=g) for _ in range(4)]
    pr = p0.clone().requires_grad_(True)
    ref = torch.optim.Adam([pr], lr=0.01)
    for gr in grads[:2]:
        pr.grad = gr.clone()
        ref.step()
    pd = pr.detach().clone().cuda().requires_grad_(True)
    ours = optim.Adam([pd], lr=0.01)
    buf = io.BytesIO()  # through a checkpoint file, as a resume would
    torch.save(ref.state_dict(), buf)
    buf.seek(0)
    ours.load_state_dict(torch.load(buf, weights_only=True))
    for gr in grads[2:]:
        pr.grad = gr.clone()
        ref.step()
        pd.grad = gr.cuda()
        ours.step()
    assert torch.allclose(pd.detach().cpu(), pr.detach(), rtol=0, atol=1e-6)


@pytest.mark.parametrize("B,I,O,deg,compute,family", [
    (8192, 1024, 1024, 8, 1, None),  # unsplit pipelined forward sums the bias; tanh in the pack launch
    (16384, 512, 512, 16, 1, None),  # the same at degree 16 (config-4 layer shape)
    (8192, 1024, 1024, 8, 0, "jacobi"),  # fp32, family basis, bias summed in the forward
    (1000, 100, 150, 6, 0, None),    # padded inputs: tanh launched on its own
    (300, 256, 200, 3, 1, None),     # split small-batch forward: bias summed by the split reduce
    (100, 16, 96, 4, 0, None),       # unsplit small-batch forward: bias summed in its epilogue
    (1024, 1024, 64, 8, 1, None),    # split pipelined forward: bias summed by the split reduce
    (20, 512, 64, 8, 1, None),       # streaming forward (tanh computed in the stream kernel)
    (2, 512, 2048, 8, 1, None),      # one-launch column-owning forward
    (64, 2048, 2048, 8, 1, None),    # streaming forward with a large output: bias by a launch
    (2048, 256, 256, 16, 1, "jacobi"),
])
def test_pack_forward_equals_pack_then_forward(B, I, O, deg, compute, family):
    """ckan_pack_forward gives the bits of ckan_pack_coeffs(_basis) followed
    by ckan_forward: y, the tanh cache and the whole packed buffer."""
    import ctypes
    from kan_amd import _lib
    lib = _lib.load()
    print(f"pack_forward B={B} I={I} O={O} deg={deg} compute={compute} family={family}", flush=True)
    g = torch.Generator().manual_seed(B + I + deg)
    x = (torch.randn(B, I, generator=g) * 1.5).cuda()
    c = (torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))).cuda()
    d = _lib.make_desc(B, I, O, deg, compute, 0)
    spec = _lib.make_spec(_lib.CKAN_BASIS_JACOBI, deg, 0.5, -0.25) if family else None
    s = _lib.stream_ptr(x.device)
    nb = lib.ckan_packed_bytes(ctypes.byref(d))
    nt = lib.ckan_tcache_elems(ctypes.byref(d))
    wsb = lib.ckan_fwd_workspace_bytes(ctypes.byref(d))
    outs = []
    for fused in (False, True):
        packed = torch.zeros(nb, dtype=torch.uint8, device="cuda")
        t = torch.zeros(nt, device="cuda")
        y = torch.zeros(B, O, device="cuda")
        ws = torch.zeros(max(wsb, 256), dtype=torch.uint8, device="cuda")
        if fused:
            _lib.check(lib.ckan_pack_forward(ctypes.byref(d), spec, c.data_ptr(), packed.data_ptr(),
                                             x.data_ptr(), y.data_ptr(), t.data_ptr(), ws.data_ptr(),
                                             wsb, s))
        else:
            if spec is None:
                _lib.check(lib.ckan_pack_coeffs(ctypes.byref(d), c.data_ptr(), packed.data_ptr(), s))
            else:
                _lib.check(lib.ckan_pack_coeffs_basis(ctypes.byref(d), spec, c.data_ptr(),
                                                      packed.data_ptr(), s))
            _lib.check(lib.ckan_forward(ctypes.byref(d), x.data_ptr(), packed.data_ptr(), y.data_ptr(),
                                        t.data_ptr(), ws.data_ptr(), wsb, s))
        torch.cuda.synchronize()
        outs.append((y, t, packed))
    (y0, t0, p0), (y1, t1, p1) = outs
    assert torch.equal(y0, y1)
    assert torch.equal(t0, t1)
    assert torch.equal(p0, p1)
    if family is None and B * I <= 4096 * 1024:
        assert _rel(y1.cpu(), orc.layer_forward(x.cpu(), c.cpu())) <= (FP32_TOL if compute == 0 else BF16_TOL)


@pytest.mark.parametrize("compute,tol", [("fp32", FP32_TOL), ("bf16", BF16_TOL)])
def test_packed_operand_cache_reuse_and_invalidation(compute, tol):
    """The drop-in layer packs its coefficients once per version of the
    parameter: a second call with C unchanged reuses the packed buffer and
    gives the bits of an uncached call; an in-place update (under no_grad, or
    an optimizer step) is packed again and matches the oracle on the new C."""
    import kan_amd
    from kan_amd import functional as F
    print(f"pack cache {compute}", flush=True)
    torch.manual_seed(5)
    layer = kan_amd.ChebyKANLayer(96, 80, 8, compute=compute).cuda()
    x = torch.randn(300, 96).cuda()
    p = layer.cheby_coeffs

    def ref(xc):
        c = p.detach().cpu()
        if compute == "bf16":
            c = c.bfloat16().float()
        return orc.layer_forward(xc.cpu(), c)

    with torch.no_grad():
        y1 = layer(x)
        e1 = F.cached_pack(p)
        y2 = layer(x)
        assert F.cached_pack(p) is e1  # reused, no re-pack
        y_fresh = F.chebykan(x, p.detach().clone(), compute)  # another tensor: packed anew
    torch.cuda.synchronize()
    assert torch.equal(y1, y2) and torch.equal(y2, y_fresh)
    assert _rel(y2, ref(x)) <= tol
    with torch.no_grad():
        p.add_(0.01 * torch.randn_like(p))
        y3 = layer(x)
    assert F.cached_pack(p) is not e1
    assert _rel(y3, ref(x)) <= tol
    # an optimizer step through autograd invalidates it as well
    opt = torch.optim.SGD(layer.parameters(), lr=0.5)
    layer(x).pow(2).sum().backward()
    e3 = F.cached_pack(p)
    opt.step()
    with torch.no_grad():
        y4 = layer(x)
    assert F.cached_pack(p) is not e3
    assert _rel(y4, ref(x)) <= tol
    # and so does a step of this package's own optimizers, which write the
    # parameter through the C-ABI (they advance its version themselves)
    from kan_amd import optim
    opt2 = optim.Adam(layer.parameters(), lr=0.05)
    layer.cheby_coeffs.grad = None
    layer(x).pow(2).sum().backward()
    e4 = F.cached_pack(p)
    opt2.step()
    with torch.no_grad():
        y5 = layer(x)
    assert F.cached_pack(p) is not e4
    assert _rel(y5, ref(x)) <= tol
    F.clear_pack_cache()
    assert F.cached_pack(p) is None
