"""GPU parity of the config-4 workload: the resident 512->512->512->512->64
ChebyKAN stack at degree 16 (kan/layers/base.py:144-166 over
kan/layers/chebykan.py:53-67), fp32 master coefficients, bf16 MFMA compute
with fp32 accumulation, MSE loss and SGD.

* At a batch the CPU oracle finishes in seconds, the executor's per-step
  losses and coefficient updates are compared with the oracle's training loop
  evaluated on bf16-rounded coefficients (the reference cannot run bf16
  coefficients itself), at the bf16 tolerance 2e-2 relative.
* The same over a 30-step trajectory (every step's loss, the total fall, and
  the coefficients' total change at 5e-2: the later steps' gradients are near
  zero, so rounding is a larger share of them).
* At the full batch (65536 rows), after 2 and after 100 steps (the
  benchmarked run), the final forward is checked on sampled rows against the
  oracle, and the loss the next step reports must equal the MSE of that
  forward (a size-independent self-consistency property).
"""
import pytest
import torch

from oracle import chebykan_oracle as orc

pytestmark = pytest.mark.gpu

WIDTHS = [512, 512, 512, 512, 64]
DEGREES = [16, 16, 16, 16]
BF16_TOL = 2e-2


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _data(B, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(B, WIDTHS[0], generator=g) * 6 - 3
    W = torch.randn(WIDTHS[0], WIDTHS[-1], generator=g) / WIDTHS[0] ** 0.5
    y = x @ W + 0.1 * torch.randn(B, WIDTHS[-1], generator=g)
    return x, y


def _coeffs(seed):
    torch.manual_seed(seed)
    return [orc.init_coeffs(WIDTHS[l], WIDTHS[l + 1], DEGREES[l]) for l in range(len(DEGREES))]


def test_config4_stack_steps_match_oracle():
    from kan_amd import ResidentExecutor
    B, steps, lr = 1024, 3, 0.01
    print(f"config 4 stack B={B} steps={steps} bf16", flush=True)
    x, y = _data(B, 41)
    coeffs = _coeffs(42)
    ex = ResidentExecutor(WIDTHS, DEGREES, B, compute="bf16", loss="mse", optimizer="sgd", lr=lr)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, yd = x.cuda(), y.cuda()
    losses = [ex.step(xd, yd).item() for _ in range(steps)]
    c_ref, losses_ref = orc.train_steps(x, y, coeffs, steps=steps, loss="mse", optimizer="sgd",
                                        lr=lr, bf16_coeffs=True)
    for k, (a, b) in enumerate(zip(losses, losses_ref)):
        assert abs(a - b) <= BF16_TOL * abs(b), (k, a, b)
    # at lr 0.01 the loss falls by ~1e-3 of itself over these steps, so the
    # comparison above hardly sees training; the fall itself must match
    drop, drop_ref = losses[0] - losses[-1], losses_ref[0] - losses_ref[-1]
    assert drop_ref > 0
    assert abs(drop - drop_ref) <= BF16_TOL * drop_ref, (drop, drop_ref)
    for l in range(len(DEGREES)):
        got = ex.get_coeffs(l).cpu() - coeffs[l]
        want = c_ref[l] - coeffs[l]
        assert want.norm() > 0
        assert _rel(got, want) <= BF16_TOL, (l, _rel(got, want))
    ex.close()


def test_config4_full_batch_forward_and_loss_consistency():
    from kan_amd import ResidentExecutor
    B, lr = 65536, 0.01
    print(f"config 4 stack full batch B={B}", flush=True)
    x, y = _data(B, 43)
    coeffs = _coeffs(44)
    ex = ResidentExecutor(WIDTHS, DEGREES, B, compute="bf16", loss="mse", optimizer="sgd", lr=lr)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, yd = x.cuda(), y.cuda()
    l0 = ex.step(xd, yd).item()
    l1 = ex.step(xd, yd).item()
    assert l1 < l0
    out = ex.forward(xd)
    cur = [ex.get_coeffs(l).cpu() for l in range(len(DEGREES))]
    # sampled rows against the oracle (fp32 math on bf16-rounded coefficients)
    rows = torch.randperm(B, generator=torch.Generator().manual_seed(45))[:256]
    ref = orc.mlp_forward(x[rows], cur, bf16_coeffs=True)
    assert _rel(out.cpu()[rows], ref) <= BF16_TOL
    # the next step's loss is the MSE of exactly this forward
    mse = torch.mean((out.double() - yd.double()) ** 2).item()
    l2 = ex.step(xd, yd).item()
    assert abs(l2 - mse) <= 1e-5 * mse, (l2, mse)
    assert torch.isfinite(out).all()
    ex.close()


def test_config4_trajectory_matches_oracle():
    """30 steps at the config's learning rate: every step's loss, the total
    fall and the coefficients' total change against the oracle's loop on
    bf16-rounded coefficients.  (At lr 0.01 this stack falls over its first
    steps and then holds; at 0.02 and above the reference's own loop
    diverges to NaN, so a longer trajectory shows no more training.)"""
    from kan_amd import ResidentExecutor
    B, steps, lr = 512, 30, 0.01
    print(f"config 4 trajectory B={B} steps={steps} lr={lr}", flush=True)
    x, y = _data(B, 47)
    coeffs = _coeffs(48)
    ex = ResidentExecutor(WIDTHS, DEGREES, B, compute="bf16", loss="mse", optimizer="sgd", lr=lr)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    losses = ex.fit(x.cuda(), y.cuda(), steps).cpu().tolist()
    c_ref, losses_ref = orc.train_steps(x, y, coeffs, steps=steps, loss="mse", optimizer="sgd",
                                        lr=lr, bf16_coeffs=True)
    assert losses_ref[-1] < losses_ref[0]
    for k, (a, b) in enumerate(zip(losses, losses_ref)):
        assert abs(a - b) <= BF16_TOL * abs(b), (k, a, b)
    drop, drop_ref = losses[0] - losses[-1], losses_ref[0] - losses_ref[-1]
    assert abs(drop - drop_ref) <= 5 * BF16_TOL * drop_ref, (drop, drop_ref)
    # once the loss holds, the steps' gradients are near zero and bf16
    # rounding is a larger share of each later increment: 5e-2 for the total
    # change over 30 steps (2e-2 holds for the first 3, in the test above)
    rels = [_rel(ex.get_coeffs(l).cpu() - coeffs[l], c_ref[l] - coeffs[l]) for l in range(len(DEGREES))]
    print("coefficient change, relative difference per layer:", rels, flush=True)
    assert max(rels) <= 5e-2, rels
    ex.close()


def test_config4_full_batch_after_100_steps():
    """The benchmarked workload itself: 100 steps at the full batch (65536
    rows), then the full-batch properties: the loss fell, the final forward
    matches the oracle on sampled rows, and the next step reports the MSE of
    exactly that forward."""
    from kan_amd import ResidentExecutor
    B, lr, steps = 65536, 0.01, 100
    print(f"config 4 stack full batch B={B}, {steps} steps", flush=True)
    x, y = _data(B, 49)
    coeffs = _coeffs(50)
    ex = ResidentExecutor(WIDTHS, DEGREES, B, compute="bf16", loss="mse", optimizer="sgd", lr=lr)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, yd = x.cuda(), y.cuda()
    losses = ex.fit(xd, yd, steps).cpu()
    assert torch.isfinite(losses).all()
    assert losses[-1] < losses[0]
    out = ex.forward(xd)
    cur = [ex.get_coeffs(l).cpu() for l in range(len(DEGREES))]
    rows = torch.randperm(B, generator=torch.Generator().manual_seed(51))[:256]
    ref = orc.mlp_forward(x[rows], cur, bf16_coeffs=True)
    assert _rel(out.cpu()[rows], ref) <= BF16_TOL
    mse = torch.mean((out.double() - yd.double()) ** 2).item()
    nxt = ex.step(xd, yd).item()
    assert abs(nxt - mse) <= 1e-5 * mse, (nxt, mse)
    ex.close()
