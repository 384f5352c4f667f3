"""CPU-side checks of the C-ABI boundary: the library loads, exports every
function include/chebykan.h declares, and rejects invalid requests on the
host before any launch (no GPU needed: these calls return before touching
the HIP runtime)."""
import ctypes
import os
import re

import pytest
import torch

from kan_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    txt = open(os.path.join(ROOT, "include", "chebykan.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(ckan_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert len(names) >= 15
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_lib.SIGNATURES) == set(names)


def test_python_constants_match_header_enums():
    """Every enum constant of include/chebykan.h that the ctypes layer mirrors
    (same name in kan_amd._lib) has the header's value."""
    txt = open(os.path.join(ROOT, "include", "chebykan.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    consts = {}
    for body in re.findall(r"typedef enum \w+ \{(.*?)\}", txt, flags=re.S):
        for name, value in re.findall(r"\b(CKAN_[A-Z0-9_]+)\s*=\s*(\d+)", body):
            consts[name] = int(value)
    assert {"CKAN_EXEC_NO_FUSED_SMALL", "CKAN_EXEC_PACK_EACH_STEP", "CKAN_LOSS_CE"} <= set(consts)
    mirrored = [n for n in consts if hasattr(_lib, n)]
    assert len(mirrored) >= 10
    for n in mirrored:
        assert getattr(_lib, n) == consts[n], n


def test_version_string():
    assert b"gfx950" in _lib.load().ckan_version()


def _desc(B=8, I=4, O=3, deg=8, compute=0, cdt=0):
    return _lib.make_desc(B, I, O, deg, compute, cdt)


@pytest.mark.parametrize("field,value,code", [
    ("batch", -1, _lib.CKAN_ERR_INVALID_ARG),
    ("in_dim", 0, _lib.CKAN_ERR_INVALID_ARG),
    ("out_dim", 0, _lib.CKAN_ERR_INVALID_ARG),
    ("degree", -1, _lib.CKAN_ERR_INVALID_ARG),
    ("degree", 1025, _lib.CKAN_ERR_UNSUPPORTED),
    ("compute", 7, _lib.CKAN_ERR_INVALID_ARG),
    ("coeff_dtype", 5, _lib.CKAN_ERR_INVALID_ARG),
    ("input_map", 1, _lib.CKAN_ERR_INVALID_ARG),   # affine with in_scale 0
    ("input_map", 7, _lib.CKAN_ERR_INVALID_ARG),
    ("in_scale", 0.5, _lib.CKAN_ERR_INVALID_ARG),  # set with the tanh map
])
def test_descriptor_validation(field, value, code):
    lib = _lib.load()
    d = _desc()
    setattr(d, field, value)
    assert lib.ckan_forward(ctypes.byref(d), 1, 1, 1, 1, None, 0, None) == code
    assert lib.ckan_last_error()
    assert lib.ckan_packed_bytes(ctypes.byref(d)) == 0


def test_high_degree_sizes_and_limits():
    """Degrees 17..1024 run on the vector-ALU kernels: the packed buffer is C
    as fp32 [I, O, D] followed, at the next 256-byte boundary, by the basis
    recurrence block (3 D + 2 floats); the input-map cache has row pitch I; no
    workspace."""
    lib = _lib.load()

    def al(n):
        return -(-n // 256) * 256

    for deg, B, I, O in [(17, 8, 4, 3), (40, 33, 70, 5), (256, 1, 2, 2), (1024, 1, 2, 2)]:
        for compute, cdt in [(0, 0), (1, 1)]:
            d = _lib.make_desc(B, I, O, deg, compute, cdt)
            D = deg + 1
            assert lib.ckan_packed_bytes(d) == al(I * O * D * 4) + al((3 * D + 2) * 4)
            assert lib.ckan_tcache_elems(d) == B * I
            assert lib.ckan_fwd_workspace_bytes(d) == 0
            assert lib.ckan_bwd_workspace_bytes(d, 1, 1) == 0
    # the vector-ALU backward puts 8 inputs per block on grid y: in_dim <= 524280
    big = _lib.make_desc(4, 524288, 2, 20, 0, 0)
    assert lib.ckan_backward(big, 256, 256, 256, 256, 256, 0, None, 0, None) == _lib.CKAN_ERR_UNSUPPORTED
    assert b"524280" in lib.ckan_last_error()
    # the affine input map (finite-domain Hermite) is served at every degree
    for deg in (16, 17, 256):
        assert lib.ckan_packed_bytes(_lib.make_desc(8, 4, 3, deg, 0, 0, (0.5, 0.1))) > 0
    assert lib.ckan_packed_bytes(_lib.make_desc(8, 4, 3, 1025, 0, 0)) == 0


def test_high_degree_family_spec_checked_before_launch():
    """Jacobi / Hermite layers above degree 16 are packed as C plus the
    family's recurrence block: the spec is validated (degree match, family,
    Jacobi parameters, finite scale) before anything is launched."""
    lib = _lib.load()
    d = _lib.make_desc(8, 4, 3, 40, 0, 0)
    ok = _lib.make_spec(_lib.CKAN_BASIS_JACOBI, 40, 0.5, 1.5, 1.0)
    # valid spec: the NULL coefficient pointer is what is rejected
    assert lib.ckan_pack_coeffs_basis(d, ok, None, 256, None) == _lib.CKAN_ERR_INVALID_ARG
    assert b"NULL" in lib.ckan_last_error()
    for bad in (_lib.make_spec(_lib.CKAN_BASIS_JACOBI, 39, 0.5, 1.5, 1.0),
                _lib.make_spec(_lib.CKAN_BASIS_JACOBI, 40, -1.0, 1.5, 1.0),
                _lib.make_spec(99, 40, 0.0, 0.0, 1.0),
                _lib.make_spec(_lib.CKAN_BASIS_HERMITE, 40, 0.0, 0.0, float("inf"))):
        assert lib.ckan_pack_coeffs_basis(d, bad, 256, 256, None) == _lib.CKAN_ERR_INVALID_ARG
        assert lib.ckan_pack_forward(d, bad, 256, 256, 256, 256, 256, None, 0, None) == \
            _lib.CKAN_ERR_INVALID_ARG
        assert lib.ckan_coeff_grad_from_chebyshev(d, bad, 256, 512, 0, None) == \
            _lib.CKAN_ERR_INVALID_ARG
        assert lib.ckan_backward_basis(d, bad, 256, 256, 256, 256, 512, None, 0, None) == \
            _lib.CKAN_ERR_INVALID_ARG
    # the same at a degree the MFMA kernels serve (the map is built first)
    d8 = _lib.make_desc(8, 4, 3, 8, 0, 0)
    for bad in (_lib.make_spec(_lib.CKAN_BASIS_JACOBI, 7, 0.5, 1.5, 1.0),
                _lib.make_spec(_lib.CKAN_BASIS_JACOBI, 8, -1.5, 0.0, 1.0)):
        assert lib.ckan_backward_basis(d8, bad, 256, 256, 256, 256, 512, None, 0, None) == \
            _lib.CKAN_ERR_INVALID_ARG
    # the materialised family basis: degree up to 1024, validated first
    big = _lib.make_spec(_lib.CKAN_BASIS_HERMITE, 1025, 0.0, 0.0, 3.0)
    assert lib.ckan_family_basis(big, 256, 4, 256, None) == _lib.CKAN_ERR_UNSUPPORTED
    assert lib.ckan_family_basis(ok, None, 4, 256, None) == _lib.CKAN_ERR_INVALID_ARG
    assert b"NULL" in lib.ckan_last_error()
    assert lib.ckan_family_basis_backward(ok, 256, 256, 0, 256, None) == 0  # n == 0: nothing to do
    # the identity map in place cannot accumulate; in place without it is a no-op
    assert lib.ckan_coeff_grad_from_chebyshev(d, ok, 256, 256, 1, None) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_coeff_grad_from_chebyshev(d, ok, 256, 256, 0, None) == 0


def test_null_pointers_rejected_before_launch():
    lib = _lib.load()
    d = _desc()
    assert lib.ckan_forward(None, 1, 1, 1, 1, None, 0, None) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_forward(ctypes.byref(d), None, 16, 16, 16, None, 0, None) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_pack_coeffs(ctypes.byref(d), None, 16, None) == _lib.CKAN_ERR_INVALID_ARG
    # misaligned packed buffer
    assert lib.ckan_pack_coeffs(ctypes.byref(d), 16, 18, None) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_adam_step(16, 16, 16, 16, 4, 0, 1e-3, 0.9, 0.999, 1e-8, 0.0, None) == \
        _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_adam_step(16, 16, 16, 16, 4, 1, 1e-3, 1.5, 0.999, 1e-8, 0.0, None) == \
        _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_sgd_step(None, None, 4, 0.1, 0.0, None) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_basis(None, 4, 3, None, None) == _lib.CKAN_ERR_INVALID_ARG


def test_workspace_too_small_is_reported():
    lib = _lib.load()
    d = _desc(B=24, I=2048, O=2048, deg=8, compute=1, cdt=1)
    need = lib.ckan_fwd_workspace_bytes(ctypes.byref(d))
    assert need > 0  # 24 rows take the split-K streaming forward (partials)
    # up to 16 rows at 2048+ outputs take the one-launch forward: no workspace
    for rows in (1, 4, 16):
        assert lib.ckan_fwd_workspace_bytes(ctypes.byref(_desc(B=rows, I=2048, O=2048, deg=8,
                                                               compute=1, cdt=1))) == 0
    rc = lib.ckan_forward(ctypes.byref(d), 16, 16, 16, 16, 16, need - 256, None)
    assert rc == _lib.CKAN_ERR_WORKSPACE
    assert b"workspace" in lib.ckan_last_error()


def test_small_backward_needs_no_dc_workspace():
    """Latency-bound layers (few rows, few (input, output) pairs) take the
    small vector-ALU dC, and with at most 64 outputs the small vector-ALU dx:
    both read dy as given, so neither needs a re-layout or split partials.
    Past 64 outputs dx takes the GEMM and its dY re-layout again."""
    lib = _lib.load()
    d = _desc(B=256, I=784, O=64, deg=4)
    assert lib.ckan_bwd_workspace_bytes(ctypes.byref(d), 0, 1) == 0
    assert lib.ckan_bwd_workspace_bytes(ctypes.byref(d), 1, 1) == 0
    assert lib.ckan_bwd_workspace_bytes(ctypes.byref(d), 1, 0) == 0
    wide = _desc(B=256, I=64, O=128, deg=4)
    assert lib.ckan_bwd_workspace_bytes(ctypes.byref(wide), 1, 0) > 0
    big = _desc(B=8192, I=1024, O=1024, deg=8, compute=1)
    assert lib.ckan_bwd_workspace_bytes(ctypes.byref(big), 0, 1) > 0


def test_small_backward_grid_limit_routes_to_gemm():
    """The small vector-ALU dx puts 8 inputs per block on grid y, the small dC
    8 outputs: past 65535 blocks (524280 inputs / outputs) a layer leaves
    those kernels for the GEMM path, which re-lays dy out in a workspace."""
    lib = _lib.load()

    def ws(B, I, O, need_dx, need_dc):
        return lib.ckan_bwd_workspace_bytes(ctypes.byref(_desc(B=B, I=I, O=O, deg=4)), need_dx, need_dc)

    assert ws(1, 524280, 2, 1, 0) == 0
    assert ws(1, 524288, 2, 1, 0) > 0
    assert ws(1, 1, 524280, 0, 1) == 0
    assert ws(1, 1, 524288, 0, 1) > 0


def test_empty_calls_are_noops():
    lib = _lib.load()
    d = _desc(B=0)
    assert lib.ckan_forward(ctypes.byref(d), None, None, None, None, None, 0, None) == _lib.CKAN_OK
    assert lib.ckan_backward(ctypes.byref(d), None, None, None, None, None, 0, None, 0, None) == _lib.CKAN_OK
    assert lib.ckan_sgd_step(None, None, 0, 0.1, 0.0, None) == _lib.CKAN_OK


def test_sizes_are_consistent():
    lib = _lib.load()
    d = _desc(B=8192, I=1024, O=1024, deg=8, compute=1)
    packed = lib.ckan_packed_bytes(ctypes.byref(d))
    # Cf + Cb in bf16 (2 x 1024*1024*8*2 bytes) plus bias partials
    assert packed >= 2 * 1024 * 1024 * 8 * 2
    assert lib.ckan_tcache_elems(ctypes.byref(d)) == 8192 * 1024
    d32 = _desc(B=8192, I=1024, O=1024, deg=8, compute=0)
    assert lib.ckan_packed_bytes(ctypes.byref(d32)) >= 2 * packed - 4096 * 1024


def test_cpu_tensors_fail_loudly():
    import kan_amd
    m = kan_amd.ChebyKANLayer(4, 3, 5)
    with pytest.raises(RuntimeError, match="ROCm device"):
        m(torch.randn(2, 4))


def test_layer_api_matches_reference_surface():
    import kan_amd
    from oracle import chebykan_oracle as orc
    torch.manual_seed(11)
    m = kan_amd.ChebyKANLayer(6, 5, 4)
    c = orc.init_coeffs(6, 5, 4, seed=11)
    assert torch.equal(m.cheby_coeffs.detach(), c)
    assert list(m.state_dict()) == ["cheby_coeffs"]
    assert m.get_coefficients() is m.cheby_coeffs
    f = m.get_analytical_form()
    assert f["type"] == "ChebyKANLayer" and f["basis"] == "Chebyshev-4"
    assert f["coefficients"].shape == (6, 5, 5)
    assert repr(m) == "ChebyKANLayer(input_dim=6, output_dim=5, degree=4)"
    assert isinstance(kan_amd.get_layer("chebykan", input_dim=2, output_dim=2, degree=3),
                      kan_amd.ChebyKANLayer)
    with pytest.raises(ValueError):
        kan_amd.get_layer("nope")
    with pytest.raises(ValueError):
        kan_amd.get_basis("nope")
    b = kan_amd.get_basis("chebyshev", degree=3)
    assert b.name == "Chebyshev-3" and b.domain == (-1, 1)
    seq = kan_amd.KANSequential(kan_amd.ChebyKANLayer(3, 4, 2), kan_amd.ChebyKANLayer(4, 2, 2))
    assert len(seq.get_analytical_form()) == 2
    with pytest.raises(ValueError):
        kan_amd.ChebyKANLayer(3, 3, 3, compute="fp8")


def test_adam_state_dict_interoperates_with_torch_optim():
    """A torch.optim.Adam checkpoint loads into kan_amd.optim.Adam (step kept as
    torch keeps it, a float tensor) and the other way round."""
    from kan_amd import optim
    p = torch.nn.Parameter(torch.randn(7))
    ref = torch.optim.Adam([p], lr=0.01)
    p.grad = torch.randn(7)
    ref.step()
    ref.step()
    q = torch.nn.Parameter(p.detach().clone())
    ours = optim.Adam([q], lr=0.01)
    ours.load_state_dict(ref.state_dict())
    st = ours.state[q]
    assert torch.is_tensor(st["step"]) and float(st["step"]) == 2.0
    assert torch.equal(st["exp_avg"], ref.state[p]["exp_avg"])
    back = torch.optim.Adam([torch.nn.Parameter(p.detach().clone())], lr=0.01)
    back.load_state_dict(ours.state_dict())
    assert float(next(iter(back.state.values()))["step"]) == 2.0


def test_basis_helpers_and_network_stubs_mirror_reference():
    import kan_amd
    b = kan_amd.ChebyshevBasis(degree=3)
    x = torch.tensor([[0.0, 0.5], [1.0, 2.0]])
    assert torch.allclose(b.normalize_domain(x, (0.0, 2.0), (-1.0, 1.0)), x - 1.0)
    assert b.to_numpy(x).shape == (2, 2)
    seq = kan_amd.KANSequential(kan_amd.ChebyKANLayer(2, 2, 2))
    with pytest.raises(NotImplementedError, match="visualization"):
        seq.visualize_network()
    with pytest.raises(NotImplementedError, match="Jacobian"):
        seq.jacobian(torch.zeros(1, 2))


def test_f64_basis_entry_points_validate_before_launch():
    """The fp64 family entry points: the recurrence block's size, NULL and
    alignment checks, and the degree limit, all on the host."""
    lib = _lib.load()
    spec = _lib.make_spec(_lib.CKAN_BASIS_HERMITE, 8, 0.0, 0.0, 3.0)
    assert lib.ckan_recurrence_bytes_f64(spec) == (3 * 9 + 2) * 8
    assert lib.ckan_recurrence_bytes_f64(_lib.make_spec(_lib.CKAN_BASIS_HERMITE, 1025, 0, 0, 3.0)) == 0
    assert lib.ckan_write_recurrence_f64(spec, None, None) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_write_recurrence_f64(spec, 12, None) == _lib.CKAN_ERR_INVALID_ARG  # misaligned
    bad = _lib.make_spec(_lib.CKAN_BASIS_JACOBI, 8, -1.5, 0.0, 1.0)
    assert lib.ckan_write_recurrence_f64(bad, 256, None) == _lib.CKAN_ERR_INVALID_ARG
    d = _lib.make_desc(8, 4, 3, 8, 0, 0)
    assert lib.ckan_forward_f64_basis(d, None, 256, 256, 256, 256, None) == _lib.CKAN_ERR_INVALID_ARG
    assert lib.ckan_backward_f64_basis(d, None, 256, 256, 256, 256, 256, 0, None) == \
        _lib.CKAN_ERR_INVALID_ARG


def test_exec_create_basis_validates_before_allocating():
    """ckan_exec_create_basis: a spec whose degree differs from the layer's,
    an invalid family parameter or an invalid affine map on the first layer
    returns before the first device allocation."""
    lib = _lib.load()
    w = (ctypes.c_int32 * 3)(6, 5, 3)
    d = (ctypes.c_int32 * 2)(4, 3)
    cfg = _lib.CkanExecConfig(2, w, d, 16, 0, _lib.CKAN_LOSS_MSE, _lib.CKAN_OPT_SGD, 0, 0.01,
                              0.9, 0.999, 1e-8, 0.0, 0)
    h = ctypes.c_void_p()

    def create(specs, aff=None):
        arr = (_lib.CkanBasisSpec * 2)(*specs)
        return lib.ckan_exec_create_basis(ctypes.byref(cfg), arr, aff, ctypes.byref(h), None)

    cheb3 = _lib.make_spec(_lib.CKAN_BASIS_CHEBYSHEV, 3)
    assert create([_lib.make_spec(_lib.CKAN_BASIS_JACOBI, 5), cheb3]) == _lib.CKAN_ERR_INVALID_ARG
    assert b"basis degree 5 != layer degree 4" in lib.ckan_last_error()
    assert create([_lib.make_spec(_lib.CKAN_BASIS_JACOBI, 4, -1.5, 0.0), cheb3]) == \
        _lib.CKAN_ERR_INVALID_ARG
    assert b"alpha" in lib.ckan_last_error()
    aff = (ctypes.c_float * 4)(0.0, 0.5, 0.0, 0.0)  # scale 0 with a shift: no input map
    assert create([_lib.make_spec(_lib.CKAN_BASIS_HERMITE, 4, 0, 0, 3.0), cheb3], aff) == \
        _lib.CKAN_ERR_INVALID_ARG
    assert not h.value
