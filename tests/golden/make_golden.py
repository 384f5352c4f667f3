"""Writes the golden fixtures in this directory from the pinned CPU oracle.

The reference (0xEodum/KAN) ships no golden vectors and was not executed; these
fixtures are produced by oracle/chebykan_oracle.py, whose functions are pinned
in tests/test_oracle.py against closed forms, brute force and finite
differences.  They freeze the oracle's outputs on fixed seeds so that
regressions in the oracle or the HIP path show up as fixture mismatches.

Usage:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import chebykan_oracle as orc  # noqa: E402

CASES = [
    # name, B, I, O, deg, seed, x_scale
    ("cfg1_like", 100, 1, 1, 8, 11, 1.0),
    ("small_deg4", 17, 6, 5, 4, 12, 1.5),
    ("small_deg8", 33, 40, 24, 8, 13, 1.0),
    ("small_deg16", 20, 16, 12, 16, 14, 2.0),
    ("odd_deg3", 9, 7, 3, 3, 15, 1.0),
]


def main() -> None:
    for name, B, I, O, deg, seed, xs in CASES:
        g = torch.Generator().manual_seed(seed)
        x = torch.randn(B, I, generator=g) * xs
        c = torch.randn(I, O, deg + 1, generator=g) / (I * (deg + 1))
        dy = torch.randn(B, O, generator=g)
        y, dx, dc = orc.layer_forward_backward(x, c, dy)
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), x=x.numpy(), c=c.numpy(),
                            dy=dy.numpy(), y=y.numpy(), dx=dx.numpy(), dc=dc.numpy())
    # Chebyshev values on a grid (fp64), T_0..T_16
    t = np.linspace(-1.0, 1.0, 33)
    np.savez_compressed(os.path.join(HERE, "cheb_T_grid.npz"), t=t,
                        T=orc.cheb_T_powersum_fp64(t, 16))
    print("wrote", len(CASES) + 1, "fixtures to", HERE)


if __name__ == "__main__":
    main()
