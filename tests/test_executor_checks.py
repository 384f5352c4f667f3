"""Host-side input checks of the resident executor (kan_amd/executor.py),
run on the CPU: every bad input raises before any library call.

The executor trains a chain of ChebyKAN layers (KANSequential,
kan/layers/base.py:144-166) with torch.nn.CrossEntropyLoss semantics for
labels (an index outside [0, C) raises; ignore_index -100 has no counterpart
in the executor's loss kernels and is rejected)."""
import pytest
import torch
import torch.nn as nn

from kan_amd import ChebyKANLayer, HermiteKANLayer, JacobiKANLayer, KANSequential
from kan_amd import _lib
from kan_amd import executor as exm


class _NoLaunch:
    """Stands in for the C library: any call means a launch was attempted."""

    def __getattr__(self, name):
        raise AssertionError(f"library call {name} reached before the input check")


def _fake(widths=(6, 5, 3), batch=4, loss="ce"):
    ex = object.__new__(exm.ResidentExecutor)
    ex.device = torch.device("cpu")
    ex.widths, ex.degrees, ex.batch = list(widths), [2] * (len(widths) - 1), batch
    ex.loss_name, ex.optimizer = loss, "sgd"
    ex._lib = _NoLaunch()
    ex._labels_checked = None
    ex._h = None
    return ex


@pytest.mark.parametrize("shape", [(3, 6), (4, 5), (4, 7), (24,), (2, 4, 6)])
def test_forward_rejects_wrong_x_shape(shape):
    with pytest.raises(RuntimeError, match="x must be"):
        _fake().forward(torch.zeros(shape))


@pytest.mark.parametrize("shape", [(3, 6), (4, 5)])
def test_step_and_fit_reject_wrong_x_shape(shape):
    ex = _fake()
    lab = torch.zeros(4, dtype=torch.int64)
    with pytest.raises(RuntimeError, match="x must be"):
        ex.step(torch.zeros(shape), lab)
    with pytest.raises(RuntimeError, match="x must be"):
        ex.fit(torch.zeros(shape), lab, 3)


def test_mse_target_shape_checked():
    ex = _fake(loss="mse")
    with pytest.raises(RuntimeError, match="target must be"):
        ex.step(torch.zeros(4, 6), torch.zeros(4, 2))


@pytest.mark.parametrize("labels,match", [
    ([0, 1, 3, 2], r"\[0, 3\)"),          # one past the last class
    ([0, -1, 1, 2], r"\[0, 3\)"),         # negative
    ([0, 1, -100, 2], "ignore_index"),    # CrossEntropyLoss's default ignore_index
    ([0, 1, 2, 99], r"\[0, 3\)"),
])
def test_step_rejects_bad_labels(labels, match):
    ex = _fake()
    with pytest.raises(ValueError, match=match):
        ex.step(torch.zeros(4, 6), torch.tensor(labels))
    with pytest.raises(ValueError, match=match):
        ex.fit(torch.zeros(4, 6), torch.tensor(labels), 2)


def test_labels_shape_and_dtype_checked():
    ex = _fake()
    with pytest.raises(RuntimeError, match="labels must be"):
        ex.step(torch.zeros(4, 6), torch.zeros(3, dtype=torch.int64))
    with pytest.raises(ValueError, match="integer"):
        ex.step(torch.zeros(4, 6), torch.zeros(4))


def test_labels_rechecked_after_in_place_change():
    """A labels tensor checked once is checked again after an in-place write
    (its version changes) and a new tensor is always checked."""
    ex = _fake()
    lab = torch.tensor([0, 1, 2, 1])
    with pytest.raises(AssertionError, match="reached"):
        ex.step(torch.zeros(4, 6), lab)  # valid: gets as far as the library
    assert ex._labels_checked is not None
    lab[2] = 3
    with pytest.raises(ValueError, match=r"\[0, 3\)"):
        ex.step(torch.zeros(4, 6), lab)
    with pytest.raises(ValueError, match="ignore_index"):
        ex.step(torch.zeros(4, 6), torch.tensor([0, -100, 1, 1]))


def test_check_labels_torch_semantics():
    """Whatever check_labels accepts, torch's CrossEntropyLoss accepts with
    every row counted; what it rejects, torch rejects or ignores."""
    y = torch.randn(4, 3)
    ok = torch.tensor([0, 2, 1, 2])
    exm.check_labels(ok, 3)
    full = nn.CrossEntropyLoss()(y, ok)
    assert torch.allclose(full, nn.CrossEntropyLoss(reduction="sum")(y, ok) / 4)
    with pytest.raises((IndexError, RuntimeError)):
        nn.CrossEntropyLoss()(y, torch.tensor([0, 3, 1, 2]))
    ign = torch.tensor([0, -100, 1, 2])
    # torch leaves the ignored row out of the mean: not what the executor computes
    assert torch.allclose(nn.CrossEntropyLoss()(y, ign),
                          nn.CrossEntropyLoss(reduction="sum")(y, ign) / 3)


def test_from_sequential_rejects_other_modules():
    torch.manual_seed(0)
    good = KANSequential(ChebyKANLayer(6, 5, 2), ChebyKANLayer(5, 3, 2))
    assert [m.output_dim for m in exm.check_sequential(good)] == [5, 3]
    with pytest.raises(ValueError, match="Tanh"):
        exm.ResidentExecutor.from_sequential(
            KANSequential(ChebyKANLayer(6, 5, 2), nn.Tanh(), ChebyKANLayer(5, 3, 2)), batch=4)
    with pytest.raises(ValueError, match="Linear"):
        exm.ResidentExecutor.from_sequential(
            KANSequential(ChebyKANLayer(6, 5, 2), nn.Linear(5, 3)), batch=4)
    mixed = KANSequential(ChebyKANLayer(6, 5, 2), JacobiKANLayer(5, 4, 3),
                          HermiteKANLayer(4, 3, 2))
    assert [m.output_dim for m in exm.check_sequential(mixed)] == [5, 4, 3]
    with pytest.raises(ValueError, match="takes 4 inputs"):
        exm.ResidentExecutor.from_sequential(
            KANSequential(ChebyKANLayer(6, 5, 2), ChebyKANLayer(4, 3, 2)), batch=4)
    with pytest.raises(ValueError, match="no layers"):
        exm.ResidentExecutor.from_sequential(KANSequential(), batch=4)


def test_layer_basis_specs_and_input_maps():
    """The per-layer basis handed to ckan_exec_create_basis: None for
    ChebyKAN; the family, parameters and scale of a Jacobi / Hermite layer;
    the finite-domain affine map (scale, shift) of a Hermite layer that has
    one, u = 2 (x - lo) / (hi - lo) - 1 (the basis then runs at scale 3)."""
    assert exm.layer_basis(ChebyKANLayer(3, 2, 4)) == (None, None)
    spec, aff = exm.layer_basis(JacobiKANLayer(3, 2, 5, alpha=0.5, beta=-0.25))
    assert (spec.family, spec.degree, spec.alpha, spec.beta, spec.scale) == (
        _lib.CKAN_BASIS_JACOBI, 5, 0.5, -0.25, 1.0)
    assert aff is None
    spec, aff = exm.layer_basis(HermiteKANLayer(3, 2, 6, scaling="probabilist"))
    assert (spec.family, spec.degree, spec.scale) == (_lib.CKAN_BASIS_HERMITE_E, 6, 3.0)
    assert aff is None
    spec, aff = exm.layer_basis(HermiteKANLayer(3, 2, 6, domain=(-2.0, 6.0)))
    assert spec.family == _lib.CKAN_BASIS_HERMITE
    a, b = aff
    for x in (-2.0, 6.0, 1.0):  # 3 (a x + b) is the reference's 6 (x - lo) / (hi - lo) - 3
        assert abs(3 * (a * x + b) - (6.0 / 8.0 * (x + 2.0) - 3.0)) < 1e-12
    # an infinite domain (or normalize_domain=False) keeps 3 tanh(x)
    assert exm.layer_basis(HermiteKANLayer(3, 2, 6, domain=(-2.0, 6.0),
                                           normalize_domain=False))[1] is None
