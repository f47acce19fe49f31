"""The 3-bit Lloyd-Max codebook the K8V3 cache layout uses for V.

Minimum-MSE 8-level quantizer of a standard normal (Lloyd's iteration; the
levels agree with Max 1960's table), scaled by 1/sqrt(block) because each
coordinate of a unit-norm block of `block` elements is ~N(0, 1/block).  The
reference takes this from ``superl8.quant.lloydmax.gaussian_codebook``
(kv_cache.py:502-507), whose values are not available; these are the
published-method values.
"""

from __future__ import annotations

import math
from functools import lru_cache

import numpy as np


def _std_normal_pdf(x: float) -> float:
    return 0.0 if math.isinf(x) else math.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def _std_normal_cdf(x: float) -> float:
    if math.isinf(x):
        return 1.0 if x > 0 else 0.0
    return 0.5 * (1.0 + math.erf(x / math.sqrt(2.0)))


@lru_cache(maxsize=None)
def lloyd_max_levels(levels: int = 8) -> tuple[float, ...]:
    """Levels of the minimum-MSE `levels`-point quantizer of N(0,1), float64,
    ascending: alternate cell boundaries at midpoints and levels at the cell
    centroids until the levels stop moving."""
    c = [-2.0 + 4.0 * i / (levels - 1) for i in range(levels)]
    for _ in range(2000):
        edges = [-math.inf] + [0.5 * (c[i] + c[i + 1]) for i in range(levels - 1)] + [math.inf]
        nxt = [(_std_normal_pdf(edges[i]) - _std_normal_pdf(edges[i + 1]))
               / (_std_normal_cdf(edges[i + 1]) - _std_normal_cdf(edges[i])) for i in range(levels)]
        done = max(abs(a - b) for a, b in zip(nxt, c)) < 1e-15
        c = nxt
        if done:
            break
    return tuple(c)


def gaussian_codebook(bits: int = 3, block: int = 128) -> np.ndarray:
    """fp32 ``[2**bits]`` ascending codebook for unit-L2-norm blocks."""
    if bits != 3:
        raise ValueError("only the 3-bit (8-level) codebook is defined")
    return (np.asarray(lloyd_max_levels(8), dtype=np.float64) / math.sqrt(block)).astype(np.float32)
