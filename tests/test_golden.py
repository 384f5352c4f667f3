"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from the pinned oracle): the oracle must reproduce them (CPU), and the HIP
path must match them within the fp32 tolerance (GPU)."""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import chebykan_oracle as orc

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = sorted(p for p in glob.glob(os.path.join(HERE, "*.npz")) if "cheb_T_grid" not in p)


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_fixtures_present():
    assert len(CASES) >= 5


@pytest.mark.parametrize("path", CASES, ids=[os.path.basename(p) for p in CASES])
def test_oracle_reproduces_golden(path):
    f = np.load(path)
    y, dx, dc = orc.layer_forward_backward(torch.from_numpy(f["x"]), torch.from_numpy(f["c"]),
                                           torch.from_numpy(f["dy"]))
    assert _rel(y.numpy(), f["y"]) <= 1e-6
    assert _rel(dx.numpy(), f["dx"]) <= 1e-6
    assert _rel(dc.numpy(), f["dc"]) <= 1e-6
    # and the fp64 restatement agrees with the stored fp32 values
    dx64, dc64 = orc.backward_fp64(f["x"], f["c"], f["dy"])
    assert _rel(orc.forward_fp64(f["x"], f["c"]), f["y"]) <= 1e-5
    assert _rel(dc64, f["dc"]) <= 1e-5


def test_cheb_grid():
    f = np.load(os.path.join(HERE, "cheb_T_grid.npz"))
    assert np.allclose(orc.cheb_T_fp64(f["t"], 16), f["T"], atol=1e-9)


@pytest.mark.gpu
@pytest.mark.parametrize("path", CASES, ids=[os.path.basename(p) for p in CASES])
def test_hip_matches_golden(path):
    from kan_amd import functional as F
    f = np.load(path)
    x = torch.from_numpy(f["x"]).cuda().requires_grad_(True)
    c = torch.from_numpy(f["c"]).cuda().requires_grad_(True)
    y = F.chebykan(x, c, "fp32")
    y.backward(torch.from_numpy(f["dy"]).cuda())
    torch.cuda.synchronize()
    assert _rel(y.detach().cpu().numpy(), f["y"]) <= 1e-5
    assert _rel(x.grad.cpu().numpy(), f["dx"]) <= 1e-5
    assert _rel(c.grad.cpu().numpy(), f["dc"]) <= 1e-5


@pytest.mark.gpu
def test_hip_basis_matches_grid():
    import kan_amd
    f = np.load(os.path.join(HERE, "cheb_T_grid.npz"))
    t = torch.from_numpy(f["t"]).float().cuda()
    out = kan_amd.ChebyshevBasis(16).basis_functions(t).cpu().numpy()
    assert np.max(np.abs(out - f["T"])) <= 1e-4
