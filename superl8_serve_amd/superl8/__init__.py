"""The ``superl8`` module interface, on the gfx950 kernels.

The reference's paged-KV code (superl8serve/engine/kv_cache.py,
superl8serve/layers/gqa_attention.py, gated_gqa_attention.py) imports the
external ``superl8`` package and looks its ops up as module attributes.  This
package provides those names with the same call signatures; after
``superl8_serve_amd.shim.install()`` it is what ``import superl8`` returns.

Ops on the cache (``quantize_kv_write_paged``, ``attn_paged_decode_cached``,
``attn_paged_decode_k8v3``) are the drop-in kernels; the codec helpers
(``quantize_i8_rowwise``, ``quant.rotation.rotate_last``, ``quant.lloydmax.*``)
run the append kernel's row arithmetic, so a K8V3 write through them stores
the bytes the fused append stores; the dense attention ops
(``attn_int8_decode`` / ``attn_int8_fwd`` / ``attn_int8_varlen``) run the
fp16-input prefill kernel.  Every function takes device tensors and raises on
host tensors: there is no CPU implementation.

Beyond the reference's names, the module also carries the ops a caller adopts
at the same seam to replace several reference launches by one: the
one-launch decode step (``attn_paged_decode_append[_k8v3]``, with the step's
shared slice plan ``attn_paged_decode_plan``) for the write-then-attend pair
of gqa_attention.py:174-190, the multi-query verify
(``attn_paged_verify[_k8v3]``) for the S decode launches of
gqa_attention.py:217-314, the sliding-window decode
(``attn_paged_decode_window[_k8v3]``) for gqa_attention.py:191-196, the fused
K8V3 append (``quantize_kv_write_paged_k8v3``) for kv_cache.py:587-626 and the
block copy (``copy_blocks``) behind copy-on-write and compaction.
"""

from __future__ import annotations

import math

import torch

from .. import ops
from ..ops import (
    attn_paged_decode_append,
    attn_paged_decode_append_k8v3,
    attn_paged_decode_cached,
    attn_paged_decode_k8v3,
    attn_paged_decode_plan,
    attn_paged_decode_window,
    attn_paged_decode_window_k8v3,
    attn_paged_verify,
    attn_paged_verify_k8v3,
    copy_blocks,
    quantize_kv_write_paged,
    quantize_kv_write_paged_k8v3,
)
from . import quant

__all__ = [
    "quantize_kv_write_paged",
    "attn_paged_decode_cached",
    "attn_paged_decode_k8v3",
    "quantize_i8_rowwise",
    "quantize_kv_cache",
    "attn_int8_decode",
    "attn_int8_fwd",
    "attn_int8_varlen",
    "quant",
    # one-launch replacements at the same seam (no reference counterpart)
    "attn_paged_decode_append",
    "attn_paged_decode_append_k8v3",
    "attn_paged_decode_plan",
    "attn_paged_decode_window",
    "attn_paged_decode_window_k8v3",
    "attn_paged_verify",
    "attn_paged_verify_k8v3",
    "quantize_kv_write_paged_k8v3",
    "copy_blocks",
]


def quantize_i8_rowwise(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric RTN int8 of fp16 rows (kv_cache.py:601): ``(q, scale)``
    with ``q`` int8 of x's shape and ``scale`` fp32 ``x.shape[:-1]``
    (``absmax / 127``; an all-zero row gets scale 0 and codes 0)."""
    return ops.quantize_rows_int8(x, rotate=False)


def quantize_kv_cache(k: torch.Tensor, v: torch.Tensor, rotate: bool = True):
    """Contiguous int8 copy of fp16 K / V ``[B, Hkv, N, D]`` (kv_cache.py:1231,
    layers/attention.py:39): ``(k_i8, k_scale, v_i8, v_scale)``, K rotated
    first when ``rotate`` (the cache's K recipe), scales ``[B, Hkv, N]``."""
    k_i8, k_sc = ops.quantize_rows_int8(k, rotate=rotate)
    v_i8, v_sc = ops.quantize_rows_int8(v, rotate=False)
    return k_i8, k_sc, v_i8, v_sc


def _scale(q: torch.Tensor, scale):
    return 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)


def attn_int8_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale=None) -> torch.Tensor:
    """Attention of ``q`` ``[B, Hq, S, D]`` over dense fp16 K / V
    ``[B, Hkv, N, D]`` with every key visible (the reference's per-row
    fallback decode, kv_cache.py:688 and gqa_attention.py:145,195)."""
    return ops.attn_fwd(q, k, v, causal=False, scale=_scale(q, scale))


def attn_int8_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, causal: bool = True, scale=None,
                  window_left: int = -1) -> torch.Tensor:
    """Prefill attention over dense fp16 ``[B, H, S, D]`` tensors
    (gqa_attention.py:122-128, gated_gqa_attention.py:56,178-191): causal is
    bottom-right aligned; ``window_left >= 0`` also hides keys more than
    ``window_left`` positions behind the query."""
    return ops.attn_fwd(q, k, v, causal=causal, scale=_scale(q, scale),
                        window_left=None if window_left is None or window_left < 0 else int(window_left))


def attn_int8_varlen(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                     cu_seqlens_k: torch.Tensor, max_seqlen_q: int, max_seqlen_k: int, *, causal: bool = True,
                     scale=None, window_left: int = -1) -> torch.Tensor:
    """Varlen prefill attention over token-major fp16 ``[T, H, D]`` tensors
    (gqa_attention.py:91-101, gated_gqa_attention.py:140)."""
    return ops.attn_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, causal=causal,
                           scale=_scale(q, scale),
                           window_left=None if window_left is None or window_left < 0 else int(window_left))

