"""Derives the coefficients of the sampler's exponential (SG_C2..SG_C5 in
specgrove_amd/csrc/sg_math.h, SGO_C2..SGO_C5 in oracle/sg_oracle.c).

e^r on |r| <= ln2/2 is approximated by 1 + r + c2 r^2 + c3 r^3 + c4 r^4 +
c5 r^5 (the first two terms fixed so that E(0) = 1 exactly).  c2..c5 minimise
the relative error: least squares of (p(r) - e^r) / e^r over 4000 Chebyshev
nodes, reweighted 60 times towards the nodes with the largest error (a
Lawson-style approach to the minimax fit), in float64, then rounded to
binary32.  Prints the binary32 coefficients as C hex literals and the
relative error of the rounded polynomial (about 1.06e-7).

Run: python oracle/fit_exp_poly.py
"""
from __future__ import annotations

import numpy as np


def fit(nodes: int = 4000, rounds: int = 60) -> np.ndarray:
    h = np.log(2.0) / 2.0
    r = h * np.cos(np.pi * (np.arange(nodes) + 0.5) / nodes)
    er = np.exp(r)
    target = (er - 1.0 - r) / er
    basis = np.stack([r ** j / er for j in range(2, 6)], axis=1)
    w = np.ones_like(r)
    c = None
    for _ in range(rounds):
        c, *_ = np.linalg.lstsq(basis * w[:, None], target * w, rcond=None)
        err = np.abs(basis @ c - target)
        w = w * (1.0 + 0.5 * err / err.max())
        w /= w.mean()
    return c


def main() -> None:
    c32 = fit().astype(np.float32)
    h = np.log(2.0) / 2.0
    r = np.linspace(-h, h, 200_001)
    p = 1.0 + r + sum(float(c32[j - 2]) * r ** j for j in range(2, 6))
    for j, v in zip(range(2, 6), c32):
        print(f"c{j} = {float(v).hex()}  ({float(v):.9g})")
    print(f"relative error of the rounded polynomial: {np.abs(p / np.exp(r) - 1).max():.3e}")


if __name__ == "__main__":
    main()
