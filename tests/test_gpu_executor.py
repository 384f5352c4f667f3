"""GPU tests of the resident executor against the CPU oracle's training loop.

Configs 2 (784->64->10, deg 4, CE, SGD) and 4-like stacks (MSE, SGD) at
sizes the oracle finishes quickly, plus the config-1 Adam loop; fp32 MFMA so
the 1e-5-class tolerances of the layer apply per step (trajectories are
compared with a looser bound because rounding differences compound).
"""
import math

import pytest
import torch

from oracle import chebykan_oracle as orc

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return ((a - b).norm() / b.norm().clamp_min(1e-30)).item()


def _make(widths, degrees, seed):
    torch.manual_seed(seed)
    return [orc.init_coeffs(widths[l], widths[l + 1], degrees[l]) for l in range(len(degrees))]


@pytest.mark.parametrize("use_graph", [False, True])
def test_config2_ce_sgd_matches_oracle(use_graph):
    from kan_amd import ResidentExecutor
    print(f"executor cfg2 graph={use_graph}", flush=True)
    widths, degrees, B = [784, 64, 10], [4, 4], 256
    g = torch.Generator().manual_seed(2)
    x = torch.rand(B, 784, generator=g) * (torch.rand(B, 784, generator=g) >= 0.8).float()
    labels = torch.randint(0, 10, (B,), generator=g)
    coeffs = _make(widths, degrees, 20)
    ex = ResidentExecutor(widths, degrees, B, compute="fp32", loss="ce", optimizer="sgd",
                          lr=0.01, use_graph=use_graph)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, ld = x.cuda(), labels.cuda()
    losses = [ex.step(xd, ld).item() for _ in range(5)]
    c_ref, losses_ref = orc.train_steps(x, labels, coeffs, steps=5, loss="ce", optimizer="sgd", lr=0.01)
    for a, b in zip(losses, losses_ref):
        assert abs(a - b) <= 1e-5 * abs(b) + 1e-6
    for l in range(2):
        assert _rel(ex.get_coeffs(l), c_ref[l]) <= 1e-5
    ex.close()


@pytest.mark.parametrize("widths,degrees,B", [
    ([40, 32, 20], [3, 4], 300),   # 20 classes: the per-row-wave loss and a separate sum
    ([24, 12], [5], 1500),         # past 1024 rows: the same
])
def test_ce_multi_block_loss_matches_oracle(widths, degrees, B):
    """Small softmax cross-entropy (up to 1024 rows, 16 classes) runs as one
    launch with its sum; larger ones as one wave per row plus a sum launch."""
    from kan_amd import ResidentExecutor
    print(f"executor ce {widths} B={B}", flush=True)
    g = torch.Generator().manual_seed(7)
    x = torch.rand(B, widths[0], generator=g) * 4 - 2
    labels = torch.randint(0, widths[-1], (B,), generator=g)
    coeffs = _make(widths, degrees, 27)
    ex = ResidentExecutor(widths, degrees, B, compute="fp32", loss="ce", optimizer="sgd", lr=0.05)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    losses = [ex.step(x.cuda(), labels.cuda()).item() for _ in range(3)]
    c_ref, losses_ref = orc.train_steps(x, labels, coeffs, steps=3, loss="ce", optimizer="sgd", lr=0.05)
    for a, b in zip(losses, losses_ref):
        assert abs(a - b) <= 1e-5 * abs(b) + 1e-6
    for l in range(len(degrees)):
        assert _rel(ex.get_coeffs(l), c_ref[l]) <= 1e-5
    ex.close()


@pytest.mark.parametrize("widths,degrees,B", [
    ([200, 48, 7], [4, 3], 123),   # rows not a multiple of the tail's 4 per block, 7 classes
    ([130, 64, 16], [2, 2], 77),   # 64 inputs (one per lane) and 16 classes, degree 2
    ([300, 64, 5], [8, 8], 200),   # degree 8: 9 coefficients per (input, class)
])
def test_fused_ce_tail_matches_oracle(widths, degrees, B):
    """The last two layers of a cross-entropy stack end in one launch: the
    first layer's split sum, the second layer's forward on the vector ALU from
    its fp32 coefficients, and each row's softmax gradient and loss (mean by a
    sum launch).  Losses and trained coefficients against the oracle; the
    library's launch record shows the tail ran."""
    from kan_amd import ResidentExecutor, _lib
    print(f"executor fused ce tail {widths} {degrees} B={B}", flush=True)
    g = torch.Generator().manual_seed(11)
    x = torch.rand(B, widths[0], generator=g) * 4 - 2
    labels = torch.randint(0, widths[-1], (B,), generator=g)
    coeffs = _make(widths, degrees, 31)
    ex = ResidentExecutor(widths, degrees, B, compute="fp32", loss="ce", optimizer="sgd", lr=0.05)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, ld = x.cuda(), labels.cuda()
    _lib.profile_enable(True)
    try:
        losses = [ex.step(xd, ld).item() for _ in range(3)]
        rep = _lib.profile_report()
    finally:
        _lib.profile_enable(False)
    assert rep.get("fwd_tail", (0,))[0] == 3, rep
    c_ref, losses_ref = orc.train_steps(x, labels, coeffs, steps=3, loss="ce", optimizer="sgd", lr=0.05)
    for a, b in zip(losses, losses_ref):
        assert abs(a - b) <= 1e-5 * abs(b) + 1e-6
    for l in range(len(degrees)):
        assert _rel(ex.get_coeffs(l), c_ref[l]) <= 1e-5
    ex.close()


def test_mse_stack_deg16_sgd_matches_oracle():
    from kan_amd import ResidentExecutor
    print("executor mse deg16 stack", flush=True)
    widths, degrees, B = [64, 64, 64, 16], [16, 16, 16], 512
    g = torch.Generator().manual_seed(4)
    x = torch.rand(B, 64, generator=g) * 6 - 3
    W = torch.randn(64, 16, generator=g) / 8
    y = x @ W + 0.1 * torch.randn(B, 16, generator=g)
    coeffs = _make(widths, degrees, 40)
    ex = ResidentExecutor(widths, degrees, B, compute="fp32", loss="mse", optimizer="sgd", lr=0.01)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    losses = [ex.step(x.cuda(), y.cuda()).item() for _ in range(4)]
    c_ref, losses_ref = orc.train_steps(x, y, coeffs, steps=4, loss="mse", optimizer="sgd", lr=0.01)
    for a, b in zip(losses, losses_ref):
        assert abs(a - b) <= 1e-5 * abs(b) + 1e-7
    for l in range(3):
        assert _rel(ex.get_coeffs(l), c_ref[l]) <= 1e-5
    ex.close()


@pytest.mark.parametrize("compute,tol", [("fp32", 1e-5), ("bf16", 2e-2)])
def test_paired_pack_with_bias_reduce_matches_oracle(compute, tol):
    """A 1024 -> 2048 layer at 512 rows forwards split-K, stores tanh(y) into
    the next layer's cache from its reduce and leaves the bias sum to a
    separate reduce launch: its pack and the next layer's run as one launch,
    followed by both bias reduces."""
    from kan_amd import ResidentExecutor
    print(f"executor paired pack + bias reduce {compute}", flush=True)
    widths, degrees, B, lr = [1024, 2048, 16], [3, 3], 512, 0.01
    g = torch.Generator().manual_seed(9)
    x = torch.rand(B, widths[0], generator=g) * 4 - 2
    y = torch.randn(B, widths[-1], generator=g)
    coeffs = _make(widths, degrees, 41)
    if compute == "bf16":
        coeffs = [c.bfloat16().float() for c in coeffs]
    ex = ResidentExecutor(widths, degrees, B, compute=compute, loss="mse", optimizer="sgd", lr=lr)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    loss = ex.step(x.cuda(), y.cuda()).item()
    c_ref, losses_ref = orc.train_steps(x, y, coeffs, steps=1, loss="mse", optimizer="sgd", lr=lr)
    assert abs(loss - losses_ref[0]) <= tol * abs(losses_ref[0])
    for l in range(2):
        # the step itself (C1 - C0 = -lr * dC) against the oracle's
        assert _rel(ex.get_coeffs(l).cpu() - coeffs[l], c_ref[l] - coeffs[l]) <= tol
    ex.close()


@pytest.mark.parametrize("compute,tol", [("fp32", 1e-5), ("bf16", 2e-2)])
def test_narrow_layer_stores_tanh_for_the_next(compute, tol):
    """A 128 -> 64 layer at 65536 rows runs the pipelined forward unsplit on its
    64-column tile and stores tanh(y) straight into the next layer's cache:
    two steps against the oracle's loop (the coefficient update after the
    first step, where one gradient is the whole change, and both losses).  The
    fp32 run is checked against the oracle evaluated in fp64: at 65536 rows
    the fp32 oracle's own rounding of the gradient sums is near 1e-5."""
    from kan_amd import ResidentExecutor
    print(f"executor narrow middle layer, 64-column tile {compute}", flush=True)
    widths, degrees, B, lr = [128, 64, 24], [8, 16], 65536, 0.05
    g = torch.Generator().manual_seed(12)
    x = torch.rand(B, widths[0], generator=g) * 4 - 2
    y = torch.randn(B, widths[-1], generator=g)
    coeffs = _make(widths, degrees, 43)
    if compute == "bf16":
        coeffs = [c.bfloat16().float() for c in coeffs]
    ex = ResidentExecutor(widths, degrees, B, compute=compute, loss="mse", optimizer="sgd", lr=lr)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, yd = x.cuda(), y.cuda()
    bf = compute == "bf16"
    # the oracle's precision: fp32 on bf16-rounded coefficients, or fp64
    xo, yo, co = (x, y, coeffs) if bf else (x.double(), y.double(), [c.double() for c in coeffs])
    losses = [ex.step(xd, yd).item()]
    c_ref, _ = orc.train_steps(xo, yo, co, steps=1, loss="mse", optimizer="sgd", lr=lr,
                               bf16_coeffs=bf)
    for l in range(2):
        assert _rel(ex.get_coeffs(l).cpu() - coeffs[l], c_ref[l] - co[l]) <= tol, l
    losses.append(ex.step(xd, yd).item())
    _, losses_ref = orc.train_steps(xo, yo, co, steps=2, loss="mse", optimizer="sgd", lr=lr,
                                    bf16_coeffs=bf)
    for k in range(2):
        assert abs(losses[k] - losses_ref[k]) <= tol * abs(losses_ref[k]), (k, losses[k], losses_ref[k])
    ex.close()


@pytest.mark.parametrize("widths,degrees,B,compute", [
    ([96, 64, 10], [4, 4], 128, "fp32"),    # dC written in place by the pipelined kernel
    ([96, 64, 10], [4, 4], 512, "fp32"),    # split dC: the split-sum kernel applies the step
    ([64, 48, 16], [15, 15], 256, "fp32"),  # fp32 degree 16: the finalize kernel applies it
    ([256, 128, 10], [8, 8], 512, "bf16"),
])
def test_sgd_weight_decay_applied_by_dc_kernels(widths, degrees, B, compute):
    """One SGD step with weight decay: C1 = C0 - lr * (g + wd * C0), where
    C0 - lr * g is the oracle's step without decay."""
    from kan_amd import ResidentExecutor
    print(f"executor sgd wd {widths} {degrees} B={B} {compute}", flush=True)
    lr, wd = 0.02, 0.5
    g = torch.Generator().manual_seed(7)
    x = torch.rand(B, widths[0], generator=g) * 4 - 2
    y = torch.randn(B, widths[-1], generator=g)
    coeffs = _make(widths, degrees, 70)
    c_ref, _ = orc.train_steps(x, y, coeffs, steps=1, loss="mse", optimizer="sgd", lr=lr)
    ex = ResidentExecutor(widths, degrees, B, compute=compute, loss="mse", optimizer="sgd",
                          lr=lr, weight_decay=wd)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    ex.step(x.cuda(), y.cuda())
    tol = 1e-5 if compute == "fp32" else 1e-3
    for l in range(len(degrees)):
        want = c_ref[l].double() - lr * wd * coeffs[l].double()
        got = ex.get_coeffs(l)
        assert _rel(got, want) <= tol, (l, _rel(got, want))
        # the decay term (relative size lr * wd = 1e-2) is far above the
        # tolerance: dropping it would fail
        assert _rel(got, c_ref[l]) > 5 * tol
    ex.close()


@pytest.mark.parametrize("widths,degrees,B,compute,loss", [
    ([96, 64, 10], [4, 4], 128, "fp32", "mse"),    # pipelined dC writes C in place
    ([96, 64, 10], [4, 4], 512, "fp32", "mse"),    # split dC: the split-sum kernel applies Adam
    ([64, 48, 16], [15, 15], 256, "fp32", "mse"),  # fp32 degree 16: the finalize kernel applies it
    ([64, 48, 16], [2, 1], 256, "fp32", "mse"),    # fp32 degree 1-2: the finalize kernel as well
    ([256, 128, 10], [8, 8], 512, "bf16", "mse"),
    ([784, 64, 10], [4, 4], 256, "fp32", "ce"),    # the config-2 shape with Adam
])
def test_adam_with_weight_decay_applied_by_dc_kernels(widths, degrees, B, compute, loss):
    """Three executor Adam steps with weight decay against torch.optim.Adam on
    the oracle's gradients: coefficients, exp_avg, exp_avg_sq and the step
    count, through every dC write path."""
    from kan_amd import ResidentExecutor
    print(f"executor adam wd {widths} {degrees} B={B} {compute} {loss}", flush=True)
    bf = compute == "bf16"
    # lr 1e-3: Adam moves every coefficient by ~lr per step, tens of times the
    # init scale 1/(in * D).  At lr 0.01 the config-2 shape drives layer-2
    # inputs past |x| = 9.01 within two steps, where the reference's backward
    # is NaN by design, and at the bf16 shape merely rounding the coefficients
    # to bf16 moves the oracle's own 3-step trajectory by 17 % (eps 0.1 x the
    # median gradient); with eps = the median gradient it moves 0.3 %.
    lr, wd, steps = 1e-3, 0.3, 3
    g = torch.Generator().manual_seed(9)
    x = torch.rand(B, widths[0], generator=g) * 4 - 2
    if loss == "mse":
        y = torch.randn(B, widths[-1], generator=g)
    else:
        y = torch.randint(0, widths[-1], (B,), generator=g)
    coeffs = _make(widths, degrees, 90)
    # eps near the gradients' scale keeps Adam's update Lipschitz in the
    # gradient, so the gradient's rounding (bf16 above all) stays visible at
    # its own size rather than as sign flips of near-zero entries
    c_sgd, _ = orc.train_steps(x, y, coeffs, steps=1, loss=loss, optimizer="sgd", lr=1.0,
                               bf16_coeffs=bf)
    g0 = [c0 - c1 for c0, c1 in zip(coeffs, c_sgd)]  # first-step gradients (lr = 1)
    eps = (1.0 if bf else 0.1) * min(float(d.abs().median()) for d in g0)
    ex = ResidentExecutor(widths, degrees, B, compute=compute, loss=loss, optimizer="adam", lr=lr,
                          eps=eps, weight_decay=wd)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, yd = x.cuda(), y.cuda()
    # step 1 at the layer's own bar (exp_avg is then exactly 0.1 * (g + wd C0)),
    # the 3-step trajectory with room for rounding differences compounding
    done = 0
    for k, tol in ((1, 2e-5 if not bf else 2e-2), (steps, 5e-4 if not bf else 3e-2)):
        while done < k:
            ex.step(xd, yd)
            done += 1
        c_ref, _, st_ref = orc.train_steps(x, y, coeffs, steps=k, loss=loss, optimizer="adam", lr=lr,
                                           weight_decay=wd, eps=eps, bf16_coeffs=bf,
                                           return_state=True)
        assert all(torch.isfinite(c).all() for c in c_ref)  # no saturation NaN in the oracle
        sd = ex.state_dict()
        assert sd["step"] == k
        for l in range(len(degrees)):
            d_got = sd[f"{l}.cheby_coeffs"].double() - coeffs[l].double()
            d_want = c_ref[l].double() - coeffs[l].double()
            assert _rel(d_got, d_want) <= tol, (k, l, "C", _rel(d_got, d_want))
            r_m = _rel(sd[f"{l}.exp_avg"], st_ref[l]["exp_avg"])
            r_v = _rel(sd[f"{l}.exp_avg_sq"], st_ref[l]["exp_avg_sq"])
            assert r_m <= tol, (k, l, "exp_avg", r_m)
            assert r_v <= 2 * tol, (k, l, "exp_avg_sq", r_v)
    ex.close()


def test_config1_adam_executor_and_checkpoint():
    from kan_amd import ResidentExecutor
    print("executor cfg1 adam", flush=True)
    x = torch.linspace(-1, 1, 100).reshape(-1, 1)
    y = torch.sin(2 * math.pi * x)
    coeffs = _make([1, 1], [8], 0)
    ex = ResidentExecutor([1, 1], [8], 100, compute="fp32", loss="mse", optimizer="adam", lr=0.01,
                          use_graph=True)
    ex.set_coeffs(0, coeffs[0])
    xd, yd = x.cuda(), y.cuda()
    for _ in range(300):
        ex.step(xd, yd)
    sd = ex.state_dict()
    assert sd["step"] == 300
    for _ in range(700):
        loss = ex.step(xd, yd)
    c_ref, losses_ref = orc.train_steps(x, y, coeffs, steps=1000, loss="mse", optimizer="adam", lr=0.01)
    assert abs(loss.item() - losses_ref[-1]) <= 1e-3 * losses_ref[0]
    assert _rel(ex.get_coeffs(0), c_ref[0]) <= 1e-3
    # resume from the checkpoint in a fresh executor: same trajectory
    ex2 = ResidentExecutor([1, 1], [8], 100, compute="fp32", loss="mse", optimizer="adam", lr=0.01)
    ex2.load_state_dict(sd)
    for _ in range(700):
        loss2 = ex2.step(xd, yd)
    assert _rel(ex2.get_coeffs(0), ex.get_coeffs(0)) <= 1e-6
    ex.close()
    ex2.close()


def test_executor_forward_matches_layers():
    import kan_amd
    from kan_amd import ResidentExecutor
    torch.manual_seed(5)
    seq = kan_amd.KANSequential(kan_amd.ChebyKANLayer(32, 48, 5), kan_amd.ChebyKANLayer(48, 8, 3))
    x = torch.randn(96, 32)
    ex = ResidentExecutor.from_sequential(seq, 96, compute="fp32")
    y = ex.forward(x.cuda()).cpu()
    y_ref = orc.mlp_forward(x, [m.cheby_coeffs.detach() for m in seq])
    assert _rel(y, y_ref) <= 1e-5
    ex.close()


def test_graph_steps_follow_the_callers_buffers():
    """Graph mode replays a graph captured on the caller's x / target when they
    are the previous step's buffers, and stages inputs otherwise: switching
    buffers and rewriting one in place must give the eager executor's losses."""
    from kan_amd import ResidentExecutor
    print("executor graph buffer switching", flush=True)
    widths, degrees, B = [48, 32, 10], [4, 3], 128
    g = torch.Generator().manual_seed(8)
    xa, xb = torch.randn(B, 48, generator=g).cuda(), torch.randn(B, 48, generator=g).cuda()
    la, lb = torch.randint(0, 10, (B,), generator=g).cuda(), torch.randint(0, 10, (B,), generator=g).cuda()
    coeffs = _make(widths, degrees, 12)
    exs = [ResidentExecutor(widths, degrees, B, compute="fp32", loss="ce", optimizer="sgd", lr=0.05,
                            use_graph=ug) for ug in (False, True)]
    for ex in exs:
        for l, c in enumerate(coeffs):
            ex.set_coeffs(l, c)
    plan = [(xa, la), (xa, la), (xa, la), (xb, lb), (xb, lb), (xa, la), (xa, la)]
    for k, (x, lab) in enumerate(plan):
        if k == 2:
            xa.mul_(0.5)  # same buffer, new contents
        if k == 6:
            xa.add_(0.25)
        eager, graph = (ex.step(x, lab).item() for ex in exs)
        assert eager == graph, (k, eager, graph)
    for l in range(2):
        assert torch.equal(exs[0].get_coeffs(l), exs[1].get_coeffs(l))
    for ex in exs:
        ex.close()


@pytest.mark.parametrize("widths,degrees,B,compute,loss,opt", [
    ([1, 1], [8], 100, "fp32", "mse", "adam"),        # config 1, the README loop
    ([8, 6, 3], [3, 5], 40, "fp32", "ce", "sgd"),      # two layers: the dx path
    ([8, 6, 3], [3, 5], 40, "bf16", "ce", "sgd"),
    ([5, 7, 4], [16, 2], 33, "fp32", "mse", "adam"),   # degree 16, Adam with weight decay
])
def test_fused_small_step_matches_oracle_and_kernel_sequence(widths, degrees, B, compute, loss, opt):
    """Stacks of at most 2^18 multiply-adds per step run each step as one
    single-workgroup launch; it must follow the oracle's training loop, and
    the per-layer kernel sequence (fused_small=False) on the same inputs."""
    from kan_amd import ResidentExecutor
    print(f"fused small step {widths} {degrees} B={B} {compute} {loss} {opt}", flush=True)
    g = torch.Generator().manual_seed(21)
    x = torch.rand(B, widths[0], generator=g) * 4 - 2
    y = (torch.randn(B, widths[-1], generator=g) if loss == "mse"
         else torch.randint(0, widths[-1], (B,), generator=g))
    coeffs = _make(widths, degrees, 22)
    wd = 0.1 if opt == "adam" and degrees[0] == 16 else 0.0
    lr = 0.01 if opt == "adam" else 0.05
    steps = 5
    bf = compute == "bf16"
    c_ref, l_ref = orc.train_steps(x, y, coeffs, steps=steps, loss=loss, optimizer=opt, lr=lr,
                                   weight_decay=wd, bf16_coeffs=bf)
    tol = 2e-2 if bf else 1e-4
    res = {}
    for fused in (True, False):
        ex = ResidentExecutor(widths, degrees, B, compute=compute, loss=loss, optimizer=opt, lr=lr,
                              weight_decay=wd, fused_small=fused)
        for l, c in enumerate(coeffs):
            ex.set_coeffs(l, c)
        xd, yd = x.cuda(), y.cuda()
        losses = [ex.step(xd, yd).item() for _ in range(steps)]
        cs = [ex.get_coeffs(l).cpu() for l in range(len(degrees))]
        for k, (a, b) in enumerate(zip(losses, l_ref)):
            assert abs(a - b) <= tol * abs(b) + 1e-7, (fused, k, a, b)
        for l in range(len(degrees)):
            d_got, d_want = cs[l].double() - coeffs[l].double(), c_ref[l].double() - coeffs[l].double()
            assert _rel(d_got, d_want) <= tol, (fused, l, _rel(d_got, d_want))
        res[fused] = cs
        ex.close()
    for l in range(len(degrees)):
        assert _rel(res[True][l] - coeffs[l], res[False][l] - coeffs[l]) <= tol


@pytest.mark.parametrize("widths,degrees,B,loss,opt", [
    ([1, 1], [8], 100, "mse", "adam"),      # one-launch steps
    ([48, 32, 10], [4, 3], 128, "ce", "sgd"),  # the per-layer kernel sequence
])
def test_fit_equals_the_step_loop(widths, degrees, B, loss, opt):
    """fit(x, y, n) issues n steps from the library: the same losses and
    coefficients, bit for bit, as n calls of step()."""
    from kan_amd import ResidentExecutor
    print(f"fit vs step loop {widths} {loss} {opt}", flush=True)
    g = torch.Generator().manual_seed(23)
    x = (torch.rand(B, widths[0], generator=g) * 4 - 2).cuda()
    y = (torch.randn(B, widths[-1], generator=g) if loss == "mse"
         else torch.randint(0, widths[-1], (B,), generator=g)).cuda()
    coeffs = _make(widths, degrees, 24)
    exs = [ResidentExecutor(widths, degrees, B, compute="fp32", loss=loss, optimizer=opt, lr=0.02)
           for _ in range(2)]
    for ex in exs:
        for l, c in enumerate(coeffs):
            ex.set_coeffs(l, c)
    looped = torch.stack([exs[0].step(x, y) for _ in range(7)])
    fitted = exs[1].fit(x, y, 7)
    assert torch.equal(looped, fitted)
    for l in range(len(degrees)):
        assert torch.equal(exs[0].get_coeffs(l), exs[1].get_coeffs(l))
    for ex in exs:
        ex.close()


# (the pair needs layer 2's inputs in whole forward super-groups: 16 at
# padded degree 4, 8 at 8, 32 at 2; classes may leave an 8-output group short)
SELF_PACK_CASES = [
    ([784, 64, 10], [4, 4], 256, "sgd", 0.0),     # config 2
    ([48, 48, 7], [3, 4], 77, "adam", 0.01),      # ragged input block, degree 3 < P, Adam + decay
    ([64, 32, 5], [8, 6], 128, "sgd", 0.02),      # padded degree 8
    ([40, 32, 3], [2, 1], 100, "sgd", 0.0),       # padded degree 2; rows padded (x mapped by launch_tanh)
]


@pytest.mark.parametrize("widths,degrees,B,opt,wd", SELF_PACK_CASES)
def test_self_packed_steps_equal_the_per_step_pack(widths, degrees, B, opt, wd):
    """Two-layer cross-entropy stacks of small layers keep their packed
    operands current from the step's dC launch (no pack launch in the step);
    the losses and coefficients must equal, bit for bit, those of the same
    executor packing at every step, eager and graph-replayed, and follow the
    oracle's loop."""
    from kan_amd import ResidentExecutor, _lib
    print(f"self-packed steps {widths} {degrees} B={B} {opt}", flush=True)
    g = torch.Generator().manual_seed(31)
    x = (torch.rand(B, widths[0], generator=g) * 4 - 2).cuda()
    lab = torch.randint(0, widths[-1], (B,), generator=g).cuda()
    coeffs = _make(widths, degrees, 32)
    lr = 0.01 if opt == "adam" else 0.05
    steps = 5
    runs = {}
    for each, ug in ((True, False), (False, False), (False, True)):
        ex = ResidentExecutor(widths, degrees, B, compute="fp32", loss="ce", optimizer=opt, lr=lr,
                              weight_decay=wd, use_graph=ug, pack_each_step=each)
        for l, c in enumerate(coeffs):
            ex.set_coeffs(l, c)
        if not ug:
            torch.cuda.synchronize()
            _lib.profile_report()
            _lib.profile_enable(True)
        losses = [ex.step(x, lab).item() for _ in range(steps)]
        if not ug:
            torch.cuda.synchronize()
            _lib.profile_enable(False)
            names = set(_lib.profile_report())
            if each:
                assert "pack2" in names, names
            else:
                assert "dc_pack" in names and not any(n.startswith("pack") for n in names), names
        runs[(each, ug)] = (losses, [ex.get_coeffs(l).cpu() for l in range(2)])
        ex.close()
    ref = runs[(True, False)]
    for key in ((False, False), (False, True)):
        assert runs[key][0] == ref[0], (key, runs[key][0], ref[0])
        for a, b in zip(runs[key][1], ref[1]):
            assert torch.equal(a, b), key
    c_ref, l_ref = orc.train_steps(x.cpu(), lab.cpu(), coeffs, steps=steps, loss="ce", optimizer=opt,
                                   lr=lr, weight_decay=wd)
    for a, b in zip(ref[0], l_ref):
        assert abs(a - b) <= 1e-5 * abs(b) + 1e-6
    for l in range(2):
        d_got = ref[1][l].double() - coeffs[l].double()
        d_want = c_ref[l].double() - coeffs[l].double()
        assert _rel(d_got, d_want) <= 1e-4


def test_self_packed_operands_follow_coefficient_writes():
    """With the per-step pack gone, set_coeffs and the executor's forward must
    leave the packed operands matching C: steps after set_coeffs (and after a
    forward call) equal those of a fresh executor given the same coefficients
    (SGD has no other state)."""
    from kan_amd import ResidentExecutor
    widths, degrees, B = [784, 64, 10], [4, 4], 256
    print("self-packed executor: set_coeffs and forward between steps", flush=True)
    g = torch.Generator().manual_seed(33)
    x = (torch.rand(B, 784, generator=g) * 2 - 1).cuda()
    lab = torch.randint(0, 10, (B,), generator=g).cuda()
    c0, c1 = _make(widths, degrees, 34), _make(widths, degrees, 35)

    def make():
        return ResidentExecutor(widths, degrees, B, compute="fp32", loss="ce", optimizer="sgd",
                                lr=0.05)
    ex = make()
    for l, c in enumerate(c0):
        ex.set_coeffs(l, c)
    for _ in range(2):
        ex.step(x, lab)
    for l, c in enumerate(c1):
        ex.set_coeffs(l, c)
    la = [ex.step(x, lab).item()]
    ex.forward(x)
    la.append(ex.step(x, lab).item())
    fresh = make()
    for l, c in enumerate(c1):
        fresh.set_coeffs(l, c)
    lb = [fresh.step(x, lab).item() for _ in range(2)]
    assert la == lb, (la, lb)
    for l in range(2):
        assert torch.equal(ex.get_coeffs(l), fresh.get_coeffs(l))
    ex.close()
    fresh.close()


def test_hidden_layers_store_tanh_into_the_next_cache():
    """At large batches a hidden layer's forward writes tanh(y) straight into
    the next layer's tanh cache (no y, no separate tanh pass).  The training
    step's loss must equal the MSE of the executor's plain forward (which
    takes the unfused path) bit for bit up to the host-side mean, and the
    step must follow the oracle."""
    from kan_amd import ResidentExecutor
    widths, degrees, B, lr = [128, 256, 256, 16], [8, 8, 8], 32768, 0.01
    print(f"executor tanh-out widths={widths} B={B}", flush=True)
    g = torch.Generator().manual_seed(61)
    x = torch.rand(B, widths[0], generator=g) * 6 - 3
    y = torch.randn(B, widths[-1], generator=g)
    torch.manual_seed(62)
    coeffs = [orc.init_coeffs(widths[l], widths[l + 1], degrees[l]) for l in range(3)]
    ex = ResidentExecutor(widths, degrees, B, compute="bf16", loss="mse", optimizer="sgd", lr=lr)
    for l, c in enumerate(coeffs):
        ex.set_coeffs(l, c)
    xd, yd = x.cuda(), y.cuda()
    out0 = ex.forward(xd)
    mse0 = torch.mean((out0.double() - yd.double()) ** 2).item()
    l0 = ex.step(xd, yd).item()
    assert abs(l0 - mse0) <= 1e-6 * mse0, (l0, mse0)
    rows = torch.randperm(B, generator=torch.Generator().manual_seed(63))[:512]
    ref = orc.mlp_forward(x[rows], coeffs, bf16_coeffs=True)
    assert _rel(out0.cpu()[rows], ref) <= 2e-2
    out1 = ex.forward(xd)
    mse1 = torch.mean((out1.double() - yd.double()) ** 2).item()
    l1 = ex.step(xd, yd).item()
    assert abs(l1 - mse1) <= 1e-6 * mse1, (l1, mse1)
    assert l1 < l0
    ex.close()


# ---- Jacobi / Hermite layers in the executor ---------------------------------

def _family_stack(kinds, widths, seed):
    """The package modules of a mixed stack, their coefficients (the oracle's
    init, times the kind's scale) and the oracle's per-layer forward
    functions.  kinds: ("cheb", deg) | ("jacobi", deg, alpha, beta) |
    ("hermite", deg, scaling, domain, init_mult)."""
    from oracle import family_oracle as fam
    from kan_amd import ChebyKANLayer, HermiteKANLayer, JacobiKANLayer, KANSequential
    torch.manual_seed(seed)
    mods, fns = [], []
    for l, k in enumerate(kinds):
        i, o, d = widths[l], widths[l + 1], k[1]
        mult = 1.0
        if k[0] == "cheb":
            m, fn = ChebyKANLayer(i, o, d), None
        elif k[0] == "jacobi":
            a, b = k[2], k[3]
            m = JacobiKANLayer(i, o, d, alpha=a, beta=b)
            fn = (lambda a, b: lambda h, c: fam.family_forward(h, c, "jacobi", a, b))(a, b)
        else:
            scaling, dom, mult = k[2], k[3], k[4]
            m = HermiteKANLayer(i, o, d, scaling=scaling, domain=dom)
            name = "hermite" if scaling == "physicist" else "hermite_e"
            fn = (lambda name, dom: lambda h, c: fam.family_forward(h, c, name, domain=dom))(name, dom)
        with torch.no_grad():
            m.get_coefficients().copy_(orc.init_coeffs(i, o, d) * mult)
        mods.append(m)
        fns.append(fn)
    return KANSequential(*mods), fns


# Stacks whose fp32 oracle trajectory agrees with its fp64 run to 1e-5 over
# the steps taken, so that the bound below tests the kernels and not the
# conditioning: the Hermite layers' H_n(3 t) reach thousands, which (at the
# reference's init scale) saturates the next tanh, where the reference's
# closed-form Chebyshev backward is 0 * inf in fp32.  Inputs lie inside the
# finite domain of a Hermite layer that has one.
FAMILY_STACKS = [
    # MFMA path: Jacobi and Hermite (3 tanh) through the change of basis
    ([20, 16, 12, 6], [("jacobi", 4, 0.5, -0.3), ("hermite", 5, "physicist", None, 0.01),
                       ("cheb", 3)], None),
    # a finite-domain Hermite first layer (affine map), He_n, and a Jacobi
    # layer above degree 16 (vector-ALU recurrence, optimizer fused)
    ([10, 14, 8, 5], [("hermite", 4, "physicist", (-2.0, 2.0), 0.02),
                      ("hermite", 3, "probabilist", None, 0.2), ("jacobi", 20, 1.0, 1.0)],
     (-2.0, 2.0)),
]


def _family_inputs(widths, x_range, loss, B, seed):
    g = torch.Generator().manual_seed(seed)
    if x_range is None:
        x = torch.randn(B, widths[0], generator=g)
    else:
        x = x_range[0] + (x_range[1] - x_range[0]) * torch.rand(B, widths[0], generator=g)
    if loss == "mse":
        tgt = torch.randn(B, widths[-1], generator=g) * 0.2
    else:
        tgt = torch.randint(0, widths[-1], (B,), generator=g)
    return x, tgt


@pytest.mark.parametrize("widths,kinds,x_range", FAMILY_STACKS)
@pytest.mark.parametrize("loss,opt", [("mse", "sgd"), ("ce", "adam")])
def test_family_stack_training_matches_oracle(widths, kinds, x_range, loss, opt):
    from kan_amd import ResidentExecutor
    print(f"executor family stack {kinds} loss={loss} opt={opt}", flush=True)
    B, steps, lr = 200, 4, (0.02 if opt == "sgd" else 0.002)
    model, fns = _family_stack(kinds, widths, 31)
    x, tgt = _family_inputs(widths, x_range, loss, B, 32)
    coeffs = [m.get_coefficients().detach().clone() for m in model]
    ex = ResidentExecutor.from_sequential(model, B, compute="fp32", loss=loss, optimizer=opt, lr=lr)
    xd, td = x.cuda(), tgt.cuda()
    losses = [ex.step(xd, td).item() for _ in range(steps)]
    c_ref, l_ref = orc.train_steps(x, tgt, coeffs, steps=steps, loss=loss, optimizer=opt, lr=lr,
                                   layer_fns=fns)
    for a, b in zip(losses, l_ref):
        assert abs(a - b) <= 1e-4 * abs(b) + 1e-6, (losses, l_ref)
    for l in range(len(kinds)):
        assert _rel(ex.get_coeffs(l), c_ref[l]) <= 1e-4, l
    # the trained stack's forward is the modules' forward on the trained coefficients
    y = ex.forward(xd)
    y_ref = orc.mlp_forward(x, c_ref, layer_fns=fns)
    assert _rel(y, y_ref) <= 1e-4
    ex.close()


def test_family_stack_bf16_and_graph_replay():
    """bf16 compute (C' = C M rounded to bf16) against the fp32 oracle at the
    bf16 bound, and graph replays bit-identical to the plain step sequence
    (SGD: Adam's first steps move every coefficient by about lr whatever the
    gradient's size, which turns bf16 rounding of near-zero gradients into
    sign flips that no bound on relative error covers)."""
    from kan_amd import ResidentExecutor
    widths, kinds, x_range = FAMILY_STACKS[0]
    print("executor family stack bf16 + graph", flush=True)
    B, steps, lr = 256, 3, 0.02
    model, fns = _family_stack(kinds, widths, 41)
    x, tgt = _family_inputs(widths, x_range, "mse", B, 42)
    coeffs = [m.get_coefficients().detach().clone() for m in model]
    runs = []
    for use_graph in (False, True):
        ex = ResidentExecutor.from_sequential(model, B, compute="bf16", loss="mse",
                                              optimizer="sgd", lr=lr, use_graph=use_graph)
        xd, td = x.cuda(), tgt.cuda()
        ls = [ex.step(xd, td).item() for _ in range(steps)]
        runs.append((ls, [ex.get_coeffs(l).cpu() for l in range(len(kinds))]))
        ex.close()
    assert runs[0][0] == runs[1][0]
    for a, b in zip(runs[0][1], runs[1][1]):
        assert torch.equal(a, b)
    c_ref, l_ref = orc.train_steps(x, tgt, coeffs, steps=steps, loss="mse", optimizer="sgd",
                                   lr=lr, layer_fns=fns)
    for a, b in zip(runs[0][0], l_ref):
        assert abs(a - b) <= 3e-2 * abs(b)
    for l in range(len(kinds)):
        assert _rel(runs[0][1][l], c_ref[l]) <= 3e-2
