"""``superl8.quant``: the rotation and Lloyd-Max codecs the cache stores
(``rotation``, ``lloydmax``) and the int8 row dequantizer."""

from __future__ import annotations

import torch

from ... import ops
from . import lloydmax, rotation

__all__ = ["rotation", "lloydmax", "dequantize_int8_rowwise"]


def dequantize_int8_rowwise(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``q * scale`` in fp32, ``scale`` broadcast against ``q`` (the
    reference's tests pass ``k_scale.unsqueeze(-1)``,
    tests/test_k8v3_cache.py:118); the value the cache's readers use."""
    ops._on_gpu("q", q, torch.int8)
    ops._on_gpu("scale", scale, torch.float32, q.device)
    return q.to(torch.float32) * scale
