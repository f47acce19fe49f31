"""``superl8.quant.lloydmax``: the 3-bit Lloyd-Max V codec of the K8V3 cache
(kv_cache.py:502-507, 606-626, 643-669, 1263-1285).

Codes are the first index minimising ``|v/norm - c_j|`` in fp32 over the
per-``block_size`` L2 norm (a zero norm stores 0 and codes of u = 0), packed
as bit planes -- the arithmetic and bytes of the fused K8V3 append.  Only
``bits=3``, ``block_size=128`` and the last dimension are supported, the
shapes the cache uses."""

from __future__ import annotations

import torch

from ... import ops
from ...codebook import gaussian_codebook as _gaussian_codebook_np

__all__ = [
    "gaussian_codebook",
    "quantize_lloydmax",
    "dequantize_lloydmax",
    "pack_indices_lowbit",
    "unpack_indices_lowbit",
    "fake_quant_lloydmax",
]


def _check(bits: int, block_size: int, dim: int) -> None:
    if bits != 3:
        raise ValueError(f"lloydmax: only 3-bit codes are supported, got bits={bits}")
    if block_size != 128:
        raise ValueError(f"lloydmax: only block_size 128 is supported, got {block_size}")
    if dim not in (-1,):
        raise ValueError(f"lloydmax: only the last dimension is supported, got dim={dim}")


def gaussian_codebook(bits: int = 3, block_size: int = 128, device=None) -> torch.Tensor:
    """fp32 ``[2**bits]`` ascending codebook for unit-norm blocks of
    ``block_size`` elements: the N(0, 1) Lloyd-Max levels / sqrt(block_size)."""
    return torch.from_numpy(_gaussian_codebook_np(bits, block_size)).to(device if device is not None else "cpu")


def quantize_lloydmax(x: torch.Tensor, bits: int = 3, block_size: int = 128, dim: int = -1, codebook=None):
    """``(codes uint8 [..., D], norms fp32 [..., D/block_size], codebook)`` of
    fp16 ``x`` (tests/test_k8v3_cache.py:71-80)."""
    _check(bits, block_size, dim)
    cb = gaussian_codebook(bits, block_size, x.device) if codebook is None else codebook
    codes, norms = ops.quantize_rows_lloydmax3(x, cb.to(torch.float32))
    return codes, norms, cb


def dequantize_lloydmax(codes: torch.Tensor, norms: torch.Tensor, codebook: torch.Tensor, block_size: int = 128,
                        dim: int = -1) -> torch.Tensor:
    """``codebook[code] * norm`` of its block, fp32 ``[..., D]``."""
    _check(3, block_size, dim)
    ops._on_gpu("codes", codes, torch.uint8)
    ops._on_gpu("norms", norms, torch.float32, codes.device)
    ops._on_gpu("codebook", codebook, torch.float32, codes.device)
    d = codes.shape[-1]
    vals = codebook.reshape(-1)[codes.long()].reshape(*codes.shape[:-1], d // block_size, block_size)
    return (vals * norms.unsqueeze(-1)).reshape(codes.shape)


def pack_indices_lowbit(codes: torch.Tensor, bits: int = 3) -> torch.Tensor:
    """Bit-plane int32 words ``[..., 3D/32]`` of uint8 codes ``[..., D]``."""
    _check(bits, 128, -1)
    return ops.pack_codes3(codes)


def unpack_indices_lowbit(packed: torch.Tensor, bits: int, d: int) -> torch.Tensor:
    """uint8 codes ``[..., d]`` of bit-plane words ``[..., 3d/32]``."""
    _check(bits, 128, -1)
    return ops.unpack_codes3(packed, d)


def fake_quant_lloydmax(x: torch.Tensor, bits: int = 3, block_size: int = 128, dim: int = -1,
                        codebook=None) -> torch.Tensor:
    """Quantize then dequantize, returned in x's dtype."""
    codes, norms, cb = quantize_lloydmax(x, bits, block_size, dim, codebook)
    return dequantize_lloydmax(codes, norms, cb.to(torch.float32), block_size, dim).to(x.dtype)
