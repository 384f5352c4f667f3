"""GPU test of the allocation-free forward (ckan_forward_noalloc) through the
C-ABI: on two calls in a row, the second with a smaller input, its outputs
(y and the tanh cache) must equal ckan_forward's with a caller workspace
bit for bit (the same kernels run on the same inputs).  A shape whose
workspace exceeds the fixed scratch must be refused before any launch.
"""
import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _run(lib, _lib, B, I, O, deg, compute, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, I, generator=g) * 1.5).cuda()
    c = (torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))).cuda()
    d = _lib.make_desc(B, I, O, deg, compute, 0)
    packed = torch.empty(lib.ckan_packed_bytes(ctypes.byref(d)), dtype=torch.uint8, device="cuda")
    s = _lib.stream_ptr(x.device)
    _lib.check(lib.ckan_pack_coeffs(ctypes.byref(d), c.data_ptr(), packed.data_ptr(), s))
    nt = lib.ckan_tcache_elems(ctypes.byref(d))
    ws_bytes = lib.ckan_fwd_workspace_bytes(ctypes.byref(d))
    assert 0 < ws_bytes <= _lib.CKAN_NOALLOC_SCRATCH_BYTES, ws_bytes  # the case uses the scratch
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    y_ref = torch.empty(B, O, device="cuda")
    t_ref = torch.empty(nt, device="cuda")
    _lib.check(lib.ckan_forward(ctypes.byref(d), x.data_ptr(), packed.data_ptr(), y_ref.data_ptr(),
                                t_ref.data_ptr(), ws.data_ptr(), ws_bytes, s))
    y = torch.full((B, O), float("nan"), device="cuda")
    t = torch.full((nt,), float("nan"), device="cuda")
    _lib.check(lib.ckan_forward_noalloc(ctypes.byref(d), x.data_ptr(), packed.data_ptr(),
                                        y.data_ptr(), t.data_ptr(), s))
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref)
    assert torch.equal(t, t_ref)
    assert torch.isfinite(y).all()


@pytest.mark.parametrize("compute", [0, 1])
def test_noalloc_forward_matches_forward_twice(compute):
    from kan_amd import _lib
    lib = _lib.load()
    print(f"noalloc forward compute={compute}: B=64 2048x2048 deg 8, then B=40 512x300 deg 5",
          flush=True)
    # first call: the config-5 shape at 64 rows (streaming split-K partials)
    _run(lib, _lib, 64, 2048, 2048, 8, compute, seed=1)
    # second call, smaller: 33..64-row streaming path on a ragged shape
    _run(lib, _lib, 40, 512, 300, 5, compute, seed=2)
    print(f"noalloc forward compute={compute}: B=300 256x200 deg 3 (split pipelined tiles)",
          flush=True)
    _run(lib, _lib, 300, 256, 200, 3, compute, seed=3)


def test_noalloc_forward_refuses_oversized_scratch():
    from kan_amd import _lib
    lib = _lib.load()
    # 64 rows x 8192 x 8192 at degree 8: the streaming partials exceed 16 MiB
    d = _lib.make_desc(64, 8192, 8192, 8, 1, 0)
    need = lib.ckan_fwd_workspace_bytes(ctypes.byref(d))
    assert need > _lib.CKAN_NOALLOC_SCRATCH_BYTES
    rc = lib.ckan_forward_noalloc(ctypes.byref(d), 16, 16, 16, 16, None)
    assert rc == _lib.CKAN_ERR_WORKSPACE
    assert b"scratch" in lib.ckan_last_error()
