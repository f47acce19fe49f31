"""``superl8.quant.rotation``: the normalized Hadamard rotation applied to K
before it is quantized (kv_cache.py:36, 594-597, 1272, 1297)."""

from __future__ import annotations

import functools
import math

import torch

from ... import ops

__all__ = ["rotate_last", "hadamard_matrix"]


def rotate_last(x: torch.Tensor) -> torch.Tensor:
    """Rotate the last axis by ``H_D / sqrt(D)`` (Sylvester order, symmetric,
    an involution): fp32 Walsh-Hadamard transform with stages h = 1 .. D/2,
    one fp32 multiply by fp32(1/sqrt(D)), one rounding to x's dtype -- the
    rotation the append kernels apply to K, so ``quantize_i8_rowwise`` of this
    equals the cache's K bytes."""
    return ops.rotate_rows(x)


@functools.lru_cache(maxsize=32)
def hadamard_matrix(d: int, device="cpu", dtype=torch.float32) -> torch.Tensor:
    """``H_d / sqrt(d)`` (Sylvester, symmetric) as a dense matrix; cached per
    (d, device, dtype), with ``cache_clear`` as dist/pipeline.py:65-70
    expects.  ``rotate_last(x)`` equals ``x @ hadamard_matrix(D)`` up to the
    fp32 summation order."""
    if d < 1 or d & (d - 1):
        raise ValueError(f"hadamard_matrix: {d} is not a power of two")
    h = torch.ones(1, 1, dtype=torch.float64)
    while h.shape[0] < d:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return (h / math.sqrt(d)).to(device=device, dtype=dtype)
