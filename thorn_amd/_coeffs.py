"""Newton-Schulz coefficient schedule and Gram restart positions, host float64.

Same mathematics as thorn.py:425-514 (Polar Express, arXiv:2505.16932):
  * each iteration fits the odd quintic p(x) = a x + b x^3 + c x^5 that equioscillates around 1
    on [max(l, cushion*u), u] (a Remez exchange on four points, solved as a 4 x 4 system);
  * with a cushion above l the quintic is rescaled so that p(l) + p(u) = 2;
  * every iteration but the last is divided by the safety factor (x -> x/(1+eps));
  * the interval then maps to [p(l), 2 - p(l)].
The Gram restart search simulates scalar Gram Newton-Schulz on a log-spaced singular-value grid
and picks the restart set with the smallest worst-case dynamic range (thorn.py:482-514); the
library runs Gram Newton-Schulz with these restarts on every non-square matrix, and settings with
no stable schedule raise the reference's ValueError.
"""
from __future__ import annotations

from functools import lru_cache
from itertools import combinations

import numpy as np
import torch

_TINY = 1e-15


def _equioscillating_quintic(lo: float, hi: float) -> tuple[float, float, float]:
    if lo / hi >= 1.0 - _TINY:
        # a degenerate interval keeps the classic quintic 15/8 x - 10/8 x^3 + 3/8 x^5, scaled to hi
        return 15.0 / 8.0 / hi, -10.0 / 8.0 / hi ** 3, 3.0 / 8.0 / hi ** 5
    # Remez exchange: p - 1 alternates sign at lo, x1, x2, hi with equal magnitude E. The interior
    # points, coefficients and E stay 0-d float64 tensors and the 4 x 4 system goes through
    # torch's LAPACK solve, as in the reference: late iterations (nearly degenerate intervals)
    # are ill-conditioned enough that other evaluation orders differ in the last bits.
    f64 = torch.float64
    x1 = (3.0 * lo + hi) / 4.0      # Python floats on the first pass, 0-d tensors afterwards
    x2 = (lo + 3.0 * hi) / 4.0
    signs = torch.tensor([-1.0, 1.0], dtype=f64)
    err, prev = float('inf'), None
    a = b = c = 1.0
    while prev is None or not prev or abs(prev - err) > _TINY:
        prev = err
        lhs = torch.tensor([
            [lo, lo ** 3.0, lo ** 5.0, 1.0],
            [x1, x1 ** 3.0, x1 ** 5.0, -1.0],
            [x2, x2 ** 3.0, x2 ** 5.0, 1.0],
            [hi, hi ** 3.0, hi ** 5.0, -1.0],
        ], dtype=f64)
        a, b, c, err = torch.linalg.solve(lhs, torch.ones(4, dtype=f64))
        # interior extrema of p: roots of p'(x) = a + 3 b x^2 + 5 c x^4
        x1, x2 = torch.sqrt((-3.0 * b + signs * (9.0 * b ** 2.0 - 20.0 * a * c) ** 0.5) / (10.0 * c))
    return float(a), float(b), float(c)


@lru_cache(maxsize=None)
def ns_coefficients(lower_bound: float, iters: int, safety_factor: float = 0.0,
                    cushion: float = 0.0) -> tuple[tuple[float, float, float], ...]:
    """(a, b, c) per Newton-Schulz iteration."""
    if not 0.0 <= lower_bound <= 1.0:
        raise AssertionError('lower_bound must be in [0, 1]')
    lo, hi = float(lower_bound), 1.0
    shrink = 1.0 + safety_factor
    out = []
    for it in range(iters):
        a, b, c = _equioscillating_quintic(max(lo, cushion * hi), hi)
        if cushion * hi > lo:
            p_lo = a * lo + b * lo ** 3 + c * lo ** 5
            p_hi = a * hi + b * hi ** 3 + c * hi ** 5
            k = 2.0 / (p_lo + p_hi)
            a, b, c = a * k, b * k, c * k
        if it < iters - 1:
            a, b, c = a / shrink, b / shrink ** 3, c / shrink ** 5
        out.append((a, b, c))
        lo = a * lo + b * lo ** 3 + c * lo ** 5
        hi = 2.0 - lo
    return tuple(out)


@lru_cache(maxsize=None)
def gram_restarts(coeffs: tuple[tuple[float, float, float], ...]) -> tuple[int, ...]:
    """Smallest stable set of Gram Newton-Schulz restart positions (raises if none is stable)."""
    sv = np.logspace(0, -10, 10000)
    shift = -4e-4
    n = len(coeffs)
    for k in range(1, n):
        best, best_set = np.inf, ()
        for combo in combinations(range(1, n), k):
            worst = 0.0
            e = sv.copy()
            q = r = None
            for j, (a, b, c) in enumerate(coeffs):
                if j == 0 or j in combo:
                    if j != 0:
                        e = e * q
                    r = e * e + shift
                    q = np.ones_like(e)
                z = a + r * (b + r * c)
                q = q * z
                r = r * z * z
                worst = max(worst, float(q.max() / q.min()))
            if worst < best:
                best, best_set = worst, combo
        if best < 1e8:
            return tuple(best_set)
    raise ValueError('No stable restarts with these parameters')
