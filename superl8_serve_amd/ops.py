"""Torch-facing ops with the signatures the reference's cache code calls on the
``superl8`` module (the drop-in boundary; call sites in
``superl8serve/engine/kv_cache.py``).

Each op checks shapes/dtypes on the host, turns tensors into pointers and
element strides, and launches the gfx950 kernels of ``libsuperl8_kv.so`` on
torch's current stream.  Outputs and scratch come from the torch caching
allocator; nothing synchronizes, so every op can be captured in a HIP graph.
CPU tensors are rejected: there is no host implementation.
"""

from __future__ import annotations

import ctypes
import math
from collections.abc import Sequence

import torch

from . import _lib

__all__ = [
    "quantize_kv_write_paged",
    "quantize_kv_write_paged_k8v3",
    "attn_paged_decode_cached",
    "attn_paged_decode_k8v3",
    "attn_paged_decode_window",
    "attn_paged_decode_window_k8v3",
    "attn_paged_decode_append",
    "attn_paged_decode_append_k8v3",
    "decode_workspace_bytes",
    "attn_paged_verify",
    "attn_paged_verify_k8v3",
    "attn_varlen",
    "attn_fwd",
    "copy_blocks",
    "rotate_rows",
    "quantize_rows_int8",
    "quantize_rows_lloydmax3",
    "pack_codes3",
    "unpack_codes3",
    "snapkv_scores",
    "snapkv_scores_paged",
    "gather_slots",
]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond: bool, msg: str, exc=ValueError) -> None:
    if not cond:
        raise exc(msg)


def _on_gpu(name: str, t: torch.Tensor, dtype: torch.dtype | None = None, device=None) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the paged-KV ops run only on the HIP device)")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if device is not None and t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _cache_geometry(k_cache: torch.Tensor) -> tuple[int, int, int, int]:
    _require(k_cache.dim() == 4, f"k_cache must be [num_blocks, num_kv_heads, block_size, head_dim], got {tuple(k_cache.shape)}")
    _require(k_cache.is_contiguous(), "k_cache must be contiguous")
    n, hkv, bs, d = k_cache.shape
    return n, hkv, bs, d


def _tokens_view(x: torch.Tensor, name: str, hkv: int, d: int) -> torch.Tensor:
    _require(x.dim() == 3 and x.shape[1] == hkv and x.shape[2] == d,
             f"{name} must be [num_tokens, {hkv}, {d}], got {tuple(x.shape)}")
    if x.stride(2) != 1:
        x = x.contiguous()
    return x


def quantize_kv_write_paged(k, v, k_cache, k_scale, v_cache, v_scale, slot_mapping) -> None:
    """Quantize-on-write of fp16 K/V ``[T, Hkv, D]`` into the int8 paged cache
    (``superl8.quantize_kv_write_paged`` at kv_cache.py:1073-1081, 1108-1116,
    288-296).  K is Hadamard-rotated then RTN int8 with an fp32 per-(token,
    head) scale; V is RTN int8.  ``slot_mapping``: int32 ``[T]`` flat slots."""
    _on_gpu("k", k, torch.float16)
    dev = k.device
    _on_gpu("v", v, torch.float16, dev)
    _on_gpu("k_cache", k_cache, torch.int8, dev)
    _on_gpu("v_cache", v_cache, torch.int8, dev)
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_scale", v_scale, torch.float32, dev)
    _on_gpu("slot_mapping", slot_mapping, torch.int32, dev)
    n, hkv, bs, d = _cache_geometry(k_cache)
    _require(v_cache.shape == k_cache.shape and v_cache.is_contiguous(), "v_cache must match k_cache")
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs] contiguous")
    _require(tuple(v_scale.shape) == (n, hkv, bs) and v_scale.is_contiguous(), "v_scale must be [N, Hkv, bs] contiguous")
    k = _tokens_view(k, "k", hkv, d)
    v = _tokens_view(v, "v", hkv, d)
    t = k.shape[0]
    _require(v.shape[0] == t, "k and v token counts differ")
    _require(slot_mapping.dim() == 1 and slot_mapping.shape[0] == t, f"slot_mapping must be [{t}]")
    if t == 0:
        return
    slot_mapping = slot_mapping.contiguous()
    lib = _lib.load()
    rc = lib.s8kv_append_int8(
        k.data_ptr(), v.data_ptr(), t, hkv, d,
        k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        slot_mapping.data_ptr(), k_cache.data_ptr(), k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(),
        n, bs, _stream(k),
    )
    _lib.check(rc, "quantize_kv_write_paged")


def quantize_kv_write_paged_k8v3(k, v, k_cache, k_scale, v_packed, v_norm, v_codebook, slot_mapping,
                                 lloyd_block: int = 128) -> None:
    """Fused K8V3 append: K as ``quantize_kv_write_paged``; V through the 3-bit
    Lloyd-Max codec into ``v_packed`` (int32 ``[N, Hkv, bs, D*3/32]``) and
    ``v_norm`` (fp32 ``[N, Hkv, bs, D/128]``).  Replaces the reference's
    ``_write_k_int8`` + ``_write_v_lloydmax3`` (kv_cache.py:587-626)."""
    _on_gpu("k", k, torch.float16)
    dev = k.device
    _on_gpu("v", v, torch.float16, dev)
    _on_gpu("k_cache", k_cache, torch.int8, dev)
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_packed", v_packed, torch.int32, dev)
    _on_gpu("v_norm", v_norm, torch.float32, dev)
    _on_gpu("v_codebook", v_codebook, torch.float32, dev)
    _on_gpu("slot_mapping", slot_mapping, torch.int32, dev)
    n, hkv, bs, d = _cache_geometry(k_cache)
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs] contiguous")
    _require(tuple(v_packed.shape) == (n, hkv, bs, d * 3 // 32) and v_packed.is_contiguous(),
             "v_packed must be [N, Hkv, bs, D*3/32] contiguous")
    _require(tuple(v_norm.shape) == (n, hkv, bs, d // lloyd_block) and v_norm.is_contiguous(),
             "v_norm must be [N, Hkv, bs, D/lloyd_block] contiguous")
    _require(v_codebook.numel() == 8 and v_codebook.is_contiguous(), "v_codebook must hold 8 contiguous entries")
    k = _tokens_view(k, "k", hkv, d)
    v = _tokens_view(v, "v", hkv, d)
    t = k.shape[0]
    _require(v.shape[0] == t and slot_mapping.dim() == 1 and slot_mapping.shape[0] == t, "token counts differ")
    if t == 0:
        return
    slot_mapping = slot_mapping.contiguous()
    lib = _lib.load()
    rc = lib.s8kv_append_k8v3(
        k.data_ptr(), v.data_ptr(), t, hkv, d,
        k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        slot_mapping.data_ptr(), k_cache.data_ptr(), k_scale.data_ptr(), v_packed.data_ptr(), v_norm.data_ptr(),
        v_codebook.data_ptr(), lloyd_block, n, bs, _stream(k),
    )
    _lib.check(rc, "quantize_kv_write_paged_k8v3")


def decode_workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_context_len: int) -> int:
    """Scratch bytes the decode ops allocate for this geometry."""
    return int(_lib.load().s8kv_decode_workspace_size(batch, num_q_heads, num_kv_heads, head_dim, max_context_len))


def _decode_prep(q, k_cache, block_table, context_lens, block_size, max_context_len):
    _on_gpu("q", q, torch.float16)
    dev = q.device
    _on_gpu("k_cache", k_cache, torch.int8, dev)
    _on_gpu("block_table", block_table, torch.int32, dev)
    _on_gpu("context_lens", context_lens, torch.int32, dev)
    n, hkv, bs, d = _cache_geometry(k_cache)
    _require(int(block_size) == bs, f"block_size {block_size} does not match the cache ({bs})")
    squeeze = False
    if q.dim() == 4:
        _require(q.shape[2] == 1, f"decode q must be [B, Hq, 1, D], got {tuple(q.shape)}")
        q3 = q[:, :, 0, :]
    else:
        _require(q.dim() == 3, f"decode q must be [B, Hq, 1, D] or [B, Hq, D], got {tuple(q.shape)}")
        q3 = q
        squeeze = True
    _require(q3.shape[2] == d, f"q head_dim {q3.shape[2]} != cache head_dim {d}")
    if q3.stride(2) != 1:
        q3 = q3.contiguous()
    b, hq = q3.shape[0], q3.shape[1]
    _require(block_table.dim() == 2 and block_table.shape[0] == b, f"block_table must be [{b}, max_blocks]")
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    _require(context_lens.dim() == 1 and context_lens.shape[0] == b, f"context_lens must be [{b}]")
    context_lens = context_lens.contiguous()
    max_context_len = int(max_context_len)
    _require(max_context_len >= 0, "max_context_len must be >= 0")
    _require(max_context_len <= block_table.shape[1] * bs,
             f"max_context_len {max_context_len} exceeds the block table capacity {block_table.shape[1] * bs}")
    out = torch.empty((b, hq, 1, d) if not squeeze else (b, hq, d), dtype=torch.float16, device=dev)
    ws_bytes = decode_workspace_bytes(b, hq, hkv, d, max_context_len)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    return q3, block_table, context_lens, out, ws, ws_bytes, (n, hkv, bs, d, b, hq), max_context_len


def attn_paged_decode_cached(q, k_cache, k_scale, v_cache, v_scale, block_table, context_lens, block_size, *,
                             max_context_len, scale):
    """Ragged-batch GQA decode over the int8 paged cache
    (``superl8.attn_paged_decode_cached``, kv_cache.py:1190-1201).

    ``q``: fp16 ``[B, Hq, 1, D]`` (a transpose view is fine).  Returns fp16
    ``[B, Hq, 1, D]``.  ``max_context_len`` only sizes the context split; every
    row is gated by its own ``context_lens`` entry."""
    q3, bt, cl, out, ws, ws_bytes, geo, max_context_len = _decode_prep(
        q, k_cache, block_table, context_lens, block_size, max_context_len)
    n, hkv, bs, d, b, hq = geo
    dev = q3.device
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_cache", v_cache, torch.int8, dev)
    _on_gpu("v_scale", v_scale, torch.float32, dev)
    _require(v_cache.shape == k_cache.shape and v_cache.is_contiguous(), "v_cache must match k_cache")
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    _require(tuple(v_scale.shape) == (n, hkv, bs) and v_scale.is_contiguous(), "v_scale must be [N, Hkv, bs]")
    if b == 0:
        return out
    lib = _lib.load()
    rc = lib.s8kv_decode_int8(
        q3.data_ptr(), b, hq, hkv, d, q3.stride(0), q3.stride(1),
        k_cache.data_ptr(), k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(), n, bs,
        bt.data_ptr(), bt.stride(0), cl.data_ptr(), max_context_len, float(scale),
        out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q3),
    )
    _lib.check(rc, "attn_paged_decode_cached")
    return out


def attn_paged_decode_window(q, k_cache, k_scale, v_cache, v_scale, block_table, context_lens, block_size, *,
                             max_context_len, window, scale):
    """``attn_paged_decode_cached`` for a sliding-window layer: row b attends
    only its last ``window`` tokens, positions ``[max(0, L - window), L)``.
    The reference reads that window back dense and decodes per row
    (gqa_attention.py:191-196 with kv_cache.py:1233-1299)."""
    q3, bt, cl, out, ws, ws_bytes, geo, max_context_len = _decode_prep(
        q, k_cache, block_table, context_lens, block_size, max_context_len)
    n, hkv, bs, d, b, hq = geo
    dev = q3.device
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_cache", v_cache, torch.int8, dev)
    _on_gpu("v_scale", v_scale, torch.float32, dev)
    _require(v_cache.shape == k_cache.shape and v_cache.is_contiguous(), "v_cache must match k_cache")
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    _require(tuple(v_scale.shape) == (n, hkv, bs) and v_scale.is_contiguous(), "v_scale must be [N, Hkv, bs]")
    _require(int(window) >= 1, f"window must be >= 1, got {window}")
    if b == 0:
        return out
    lib = _lib.load()
    rc = lib.s8kv_decode_window_int8(
        q3.data_ptr(), b, hq, hkv, d, q3.stride(0), q3.stride(1),
        k_cache.data_ptr(), k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(), n, bs,
        bt.data_ptr(), bt.stride(0), cl.data_ptr(), max_context_len, int(window), float(scale),
        out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q3),
    )
    _lib.check(rc, "attn_paged_decode_window")
    return out


def attn_paged_decode_plan(k_cache, block_table, context_lens, block_size, *, num_q_heads, max_context_len,
                           layout: str = "int8", fused: bool = True, adaptive: bool = False, plan=None):
    """Slice plan of one decode step, shared by its per-layer launches.

    Every layer of a step decodes the same rows: the same ``block_table`` and
    ``context_lens``, so the same split of the token stream over the
    workgroups.  This launch computes that split once (and the storage rows
    of every workgroup's first tiles) into a small int32 device tensor;
    ``attn_paged_decode_append(..., plan=)`` / ``attn_paged_decode_append_k8v3(
    ..., plan=)`` read it instead of recomputing it.  ``k_cache`` is any
    layer's cache (geometry only); ``layout`` "int8" or "k8v3"; ``fused``
    the one-launch step ops.  Capturable (no host synchronization).

    ``adaptive``: the split follows the last step's measured workgroup times
    instead of the fixed formula.  The launches reading the plan record each
    workgroup's start and end in it; the next adaptive plan made into the
    same tensor (pass it back as ``plan``) moves the slice bounds a quarter
    of the way towards equal finish times, falling back to the formula when the
    geometry changed, the lengths moved by more than a sixteenth, or the
    times are missing.  Same cache bytes as the fixed split; outputs differ
    from it only by the rounding of the split rows' combine.  ``plan``: a
    tensor from an earlier call to write into (reused as is), else a new one
    (zeroed when adaptive)."""
    dev = k_cache.device
    _on_gpu("k_cache", k_cache, torch.int8, dev)
    _on_gpu("block_table", block_table, torch.int32, dev)
    _on_gpu("context_lens", context_lens, torch.int32, dev)
    _require(layout in ("int8", "k8v3"), f"layout must be 'int8' or 'k8v3', got {layout!r}")
    n, hkv, bs, d = _cache_geometry(k_cache)
    _require(int(block_size) == bs, f"block_size {block_size} does not match the cache ({bs})")
    _require(block_table.dim() == 2 and block_table.stride(1) == 1, "block_table must be a [B, max_blocks] tensor "
             "with unit stride on its last dim (the decode ops are then given the same tensor)")
    b = block_table.shape[0]
    _require(context_lens.dim() == 1 and context_lens.shape[0] == b and context_lens.is_contiguous(),
             f"context_lens must be a contiguous [{b}] tensor")
    lib = _lib.load()
    nbytes = int(lib.s8kv_decode_plan_size(hkv))
    if plan is None:
        plan = (torch.zeros if adaptive else torch.empty)(nbytes // 4, dtype=torch.int32, device=dev)
    else:
        _on_gpu("plan", plan, torch.int32, dev)
        _require(plan.is_contiguous() and plan.numel() * 4 >= nbytes,
                 f"plan must be a contiguous int32 tensor of at least {nbytes // 4} elements")
        nbytes = plan.numel() * 4
    entry = lib.s8kv_decode_plan_adaptive if adaptive else lib.s8kv_decode_plan
    rc = entry(b, int(num_q_heads), hkv, d, 1 if layout == "k8v3" else 0, 1 if fused else 0, n, bs,
               block_table.data_ptr(), block_table.stride(0), context_lens.data_ptr(), int(max_context_len),
               plan.data_ptr(), nbytes, _stream(k_cache))
    _lib.check(rc, "attn_paged_decode_plan")
    return plan


def _plan_args(plan, dev):
    """(pointer, bytes) of a plan tensor, for the planned C entry points
    (which reject a plan smaller than the geometry needs)."""
    _on_gpu("plan", plan, torch.int32, dev)
    _require(plan.is_contiguous(), "plan must be contiguous")
    return plan.data_ptr(), plan.numel() * 4


def attn_paged_decode_append(q, k_new, v_new, k_cache, k_scale, v_cache, v_scale, block_table, context_lens,
                             block_size, *, max_context_len, scale, plan=None):
    """One decode step of a layer in one launch: append row b's new token at
    position ``context_lens[b] - 1`` of its block table, then attend over
    positions ``0 .. context_lens[b] - 1``.

    Same cache bytes as ``quantize_kv_write_paged`` at those slots followed by
    ``attn_paged_decode_cached`` (the pair ``write_decode_static`` +
    ``decode_attn_static`` runs, kv_cache.py:1103-1116 and 1190-1201), and the
    same output.  ``k_new``, ``v_new``: fp16 ``[B, Hkv, D]``.  Rows with
    ``context_lens[b] == 0`` or ``> max_context_len`` append nothing.  The
    block receiving a row's new token must not be read by another row of the
    same call (a block being appended to is owned by its sequence).

    ``plan``: the step's slice plan from ``attn_paged_decode_plan`` (made from
    these ``block_table`` and ``context_lens`` tensors, unchanged since); the
    launch then skips locating its work and issues its first loads at once.
    Same bytes and outputs as without it; a plan made for another geometry
    or other tensors is ignored."""
    q3, bt, cl, out, ws, ws_bytes, geo, max_context_len = _decode_prep(
        q, k_cache, block_table, context_lens, block_size, max_context_len)
    n, hkv, bs, d, b, hq = geo
    dev = q3.device
    _on_gpu("k_new", k_new, torch.float16, dev)
    _on_gpu("v_new", v_new, torch.float16, dev)
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_cache", v_cache, torch.int8, dev)
    _on_gpu("v_scale", v_scale, torch.float32, dev)
    _require(v_cache.shape == k_cache.shape and v_cache.is_contiguous(), "v_cache must match k_cache")
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    _require(tuple(v_scale.shape) == (n, hkv, bs) and v_scale.is_contiguous(), "v_scale must be [N, Hkv, bs]")
    k_new = _tokens_view(k_new, "k_new", hkv, d)
    v_new = _tokens_view(v_new, "v_new", hkv, d)
    _require(k_new.shape[0] == b and v_new.shape[0] == b, f"k_new and v_new must be [{b}, {hkv}, {d}]")
    if b == 0:
        return out
    lib = _lib.load()
    args = (
        q3.data_ptr(), b, hq, hkv, d, q3.stride(0), q3.stride(1),
        k_new.data_ptr(), k_new.stride(0), k_new.stride(1), v_new.data_ptr(), v_new.stride(0), v_new.stride(1),
        k_cache.data_ptr(), k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(), n, bs,
        bt.data_ptr(), bt.stride(0), cl.data_ptr(), max_context_len, float(scale),
        out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q3),
    )
    if plan is None:
        rc = lib.s8kv_decode_append_int8(*args)
    else:
        rc = lib.s8kv_decode_append_int8_planned(*args, *_plan_args(plan, dev))
    _lib.check(rc, "attn_paged_decode_append")
    return out


def attn_paged_decode_append_k8v3(q, k_new, v_new, k_cache, k_scale, v_packed, v_norm, v_codebook, block_table,
                                  context_lens, block_size, *, max_context_len, scale, lloyd_block: int = 128,
                                  plan=None):
    """``attn_paged_decode_append`` for the K8V3 layout: row b's new token is
    written at position ``context_lens[b] - 1`` exactly as
    ``quantize_kv_write_paged_k8v3`` writes it (int8 K; 3-bit Lloyd-Max V
    words and block norms), then the row attends as ``attn_paged_decode_k8v3``
    does -- one launch for the pair the reference runs as its K8V3 write
    (kv_cache.py:587-626) and ``decode_attn_static`` (kv_cache.py:1167-1182).
    ``plan``: as for ``attn_paged_decode_append`` (made with layout "k8v3")."""
    q3, bt, cl, out, ws, ws_bytes, geo, max_context_len = _decode_prep(
        q, k_cache, block_table, context_lens, block_size, max_context_len)
    n, hkv, bs, d, b, hq = geo
    dev = q3.device
    _on_gpu("k_new", k_new, torch.float16, dev)
    _on_gpu("v_new", v_new, torch.float16, dev)
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_packed", v_packed, torch.int32, dev)
    _on_gpu("v_norm", v_norm, torch.float32, dev)
    _on_gpu("v_codebook", v_codebook, torch.float32, dev)
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    _require(tuple(v_packed.shape) == (n, hkv, bs, d * 3 // 32) and v_packed.is_contiguous(),
             "v_packed must be [N, Hkv, bs, D*3/32]")
    _require(tuple(v_norm.shape) == (n, hkv, bs, d // lloyd_block) and v_norm.is_contiguous(),
             "v_norm must be [N, Hkv, bs, D/lloyd_block]")
    _require(v_codebook.numel() == 8 and v_codebook.is_contiguous(), "v_codebook must hold 8 contiguous entries")
    k_new = _tokens_view(k_new, "k_new", hkv, d)
    v_new = _tokens_view(v_new, "v_new", hkv, d)
    _require(k_new.shape[0] == b and v_new.shape[0] == b, f"k_new and v_new must be [{b}, {hkv}, {d}]")
    if b == 0:
        return out
    lib = _lib.load()
    args = (
        q3.data_ptr(), b, hq, hkv, d, q3.stride(0), q3.stride(1),
        k_new.data_ptr(), k_new.stride(0), k_new.stride(1), v_new.data_ptr(), v_new.stride(0), v_new.stride(1),
        k_cache.data_ptr(), k_scale.data_ptr(), v_packed.data_ptr(), v_norm.data_ptr(), v_codebook.data_ptr(),
        lloyd_block, n, bs, bt.data_ptr(), bt.stride(0), cl.data_ptr(), max_context_len, float(scale),
        out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q3),
    )
    if plan is None:
        rc = lib.s8kv_decode_append_k8v3(*args)
    else:
        rc = lib.s8kv_decode_append_k8v3_planned(*args, *_plan_args(plan, dev))
    _lib.check(rc, "attn_paged_decode_append_k8v3")
    return out


def attn_paged_decode_k8v3(q, k_cache, k_scale, v_packed, v_norm, v_codebook, block_table, context_lens, block_size,
                           *, max_context_len, scale):
    """Decode over the K8V3 cache with the 3-bit V dequantized in-kernel
    (``superl8.attn_paged_decode_k8v3``, kv_cache.py:1170-1182; positional
    order pinned by tests/test_k8v3_cache.py:179-186)."""
    q3, bt, cl, out, ws, ws_bytes, geo, max_context_len = _decode_prep(
        q, k_cache, block_table, context_lens, block_size, max_context_len)
    n, hkv, bs, d, b, hq = geo
    dev = q3.device
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_packed", v_packed, torch.int32, dev)
    _on_gpu("v_norm", v_norm, torch.float32, dev)
    _on_gpu("v_codebook", v_codebook, torch.float32, dev)
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    _require(tuple(v_packed.shape) == (n, hkv, bs, d * 3 // 32) and v_packed.is_contiguous(),
             "v_packed must be [N, Hkv, bs, D*3/32]")
    lloyd_block = d // v_norm.shape[-1] if v_norm.dim() == 4 and v_norm.shape[-1] > 0 else 0
    _require(tuple(v_norm.shape[:3]) == (n, hkv, bs) and v_norm.is_contiguous(), "v_norm must be [N, Hkv, bs, D/128]")
    _require(v_codebook.numel() == 8 and v_codebook.is_contiguous(), "v_codebook must hold 8 contiguous entries")
    if b == 0:
        return out
    lib = _lib.load()
    rc = lib.s8kv_decode_k8v3(
        q3.data_ptr(), b, hq, hkv, d, q3.stride(0), q3.stride(1),
        k_cache.data_ptr(), k_scale.data_ptr(), v_packed.data_ptr(), v_norm.data_ptr(), v_codebook.data_ptr(),
        lloyd_block, n, bs, bt.data_ptr(), bt.stride(0), cl.data_ptr(), max_context_len, float(scale),
        out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q3),
    )
    _lib.check(rc, "attn_paged_decode_k8v3")
    return out


def attn_paged_decode_window_k8v3(q, k_cache, k_scale, v_packed, v_norm, v_codebook, block_table, context_lens,
                                  block_size, *, max_context_len, window, scale):
    """``attn_paged_decode_k8v3`` for a sliding-window layer: row b attends
    only its last ``window`` tokens (see ``attn_paged_decode_window``)."""
    q3, bt, cl, out, ws, ws_bytes, geo, max_context_len = _decode_prep(
        q, k_cache, block_table, context_lens, block_size, max_context_len)
    n, hkv, bs, d, b, hq = geo
    dev = q3.device
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("v_packed", v_packed, torch.int32, dev)
    _on_gpu("v_norm", v_norm, torch.float32, dev)
    _on_gpu("v_codebook", v_codebook, torch.float32, dev)
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    _require(tuple(v_packed.shape) == (n, hkv, bs, d * 3 // 32) and v_packed.is_contiguous(),
             "v_packed must be [N, Hkv, bs, D*3/32]")
    lloyd_block = d // v_norm.shape[-1] if v_norm.dim() == 4 and v_norm.shape[-1] > 0 else 0
    _require(tuple(v_norm.shape[:3]) == (n, hkv, bs) and v_norm.is_contiguous(), "v_norm must be [N, Hkv, bs, D/128]")
    _require(v_codebook.numel() == 8 and v_codebook.is_contiguous(), "v_codebook must hold 8 contiguous entries")
    _require(int(window) >= 1, f"window must be >= 1, got {window}")
    if b == 0:
        return out
    lib = _lib.load()
    rc = lib.s8kv_decode_window_k8v3(
        q3.data_ptr(), b, hq, hkv, d, q3.stride(0), q3.stride(1),
        k_cache.data_ptr(), k_scale.data_ptr(), v_packed.data_ptr(), v_norm.data_ptr(), v_codebook.data_ptr(),
        lloyd_block, n, bs, bt.data_ptr(), bt.stride(0), cl.data_ptr(), max_context_len, int(window), float(scale),
        out.data_ptr(), ws.data_ptr() if ws is not None else None, ws_bytes, _stream(q3),
    )
    _lib.check(rc, "attn_paged_decode_window_k8v3")
    return out


def _verify_inputs(q, k_cache, k_scale, block_table, prefix_lens, block_size, query_lens, tree_mask,
                   max_context_len):
    """Checks and views shared by both cache layouts; returns the prepared
    arguments and the output tensor."""
    _on_gpu("q", q, torch.float16)
    dev = q.device
    _on_gpu("k_cache", k_cache, torch.int8, dev)
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    _on_gpu("block_table", block_table, torch.int32, dev)
    _on_gpu("prefix_lens", prefix_lens, torch.int32, dev)
    n, hkv, bs, d = _cache_geometry(k_cache)
    _require(int(block_size) == bs, f"block_size {block_size} does not match the cache ({bs})")
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    _require(q.dim() == 4 and q.shape[3] == d, f"verify q must be [B, Hq, S, {d}], got {tuple(q.shape)}")
    if q.stride(3) != 1:
        q = q.contiguous()
    b, hq, s_, _ = q.shape
    _require(block_table.dim() == 2 and block_table.shape[0] == b, f"block_table must be [{b}, max_blocks]")
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    _require(prefix_lens.dim() == 1 and prefix_lens.shape[0] == b, f"prefix_lens must be [{b}]")
    prefix_lens = prefix_lens.contiguous()
    ql_ptr = None
    if query_lens is not None:
        _on_gpu("query_lens", query_lens, torch.int32, dev)
        _require(query_lens.dim() == 1 and query_lens.shape[0] == b, f"query_lens must be [{b}]")
        query_lens = query_lens.contiguous()
        ql_ptr = query_lens.data_ptr()
    tm_ptr = None
    if tree_mask is not None:
        _on_gpu("tree_mask", tree_mask, torch.int64, dev)
        _require(tuple(tree_mask.shape) == (b, s_), f"tree_mask must be int64 [{b}, {s_}]")
        _require(s_ <= 64, "tree verify supports at most 64 drafts per row")
        tree_mask = tree_mask.contiguous()
        tm_ptr = tree_mask.data_ptr()
    max_context_len = int(max_context_len)
    _require(0 <= max_context_len <= block_table.shape[1] * bs,
             f"max_context_len {max_context_len} exceeds the block table capacity {block_table.shape[1] * bs}")
    out = torch.empty((b, hq, s_, d), dtype=torch.float16, device=dev)
    # partials of a key-range split (few query blocks or very long rows)
    ws_bytes = int(_lib.load().s8kv_verify_workspace_size(b, hq, hkv, d, s_, max_context_len)) if b and s_ else 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
    # keep the contiguous copies alive until the launch is enqueued
    keep = (q, block_table, prefix_lens, query_lens, tree_mask, ws)
    head = (q.data_ptr(), b, hq, hkv, d, s_, q.stride(0), q.stride(1), q.stride(2))
    tail = (block_table.data_ptr(), block_table.stride(0), prefix_lens.data_ptr(), ql_ptr, tm_ptr, max_context_len)
    workspace = (ws.data_ptr() if ws is not None else None, ws_bytes)
    return keep, head, tail, workspace, (n, hkv, bs, d), out


def _fresh_drafts(k_draft, v_draft, b, s_, hkv, d, dev):
    """(keep-alive tensors, C arguments) of the window verify's fresh drafts:
    K rotated on the row kernel in fp32 (the kernel splits it into fp16
    hi + lo), V fp16, both ``[B, S, Hkv, D]`` with 16-byte rows."""
    if k_draft is None and v_draft is None:
        return (), (None, 0, 0, 0, None, 0, 0, 0)
    _require(k_draft is not None and v_draft is not None, "k_draft and v_draft go together")
    for name, t in (("k_draft", k_draft), ("v_draft", v_draft)):
        _on_gpu(name, t, torch.float16, dev)
        _require(tuple(t.shape) == (b, s_, hkv, d), f"{name} must be [{b}, {s_}, {hkv}, {d}] (the layer's [B, S, Hkv, D])")
    kr = rotate_rows(k_draft.float())  # contiguous fp32, rotated as the cache's K is
    vd = v_draft
    if vd.stride(3) != 1 or vd.data_ptr() % 16 or any(x % 8 for x in vd.stride()[:3]):
        vd = vd.contiguous()
    return (kr, vd), (kr.data_ptr(), kr.stride(0), kr.stride(1), kr.stride(2), vd.data_ptr(), vd.stride(0),
                      vd.stride(1), vd.stride(2))


def attn_paged_verify(q, k_cache, k_scale, v_cache, v_scale, block_table, prefix_lens, block_size, *,
                      query_lens=None, tree_mask=None, max_context_len, scale, window=None, k_draft=None,
                      v_draft=None):
    """Multi-query attention of draft / chunk queries over the int8 paged cache.

    ``q``: fp16 ``[B, Hq, S, D]`` (any strides with D contiguous, e.g. the
    ``[B, S, Hq, D] -> [B, Hq, S, D]`` transpose view).  Row b's S drafts sit
    at cache positions ``prefix_lens[b] ..`` (appended beforehand).  Query s
    sees the prefix plus draft i when ``i <= s`` (``tree_mask`` None: chain
    verify, gqa_attention.py:217-292, and bottom-right causal chunked prefill,
    gqa_attention.py:105-129) or when bit i of ``tree_mask[b, s]`` (int64
    ``[B, S]``) is set (tree verify).  Queries ``s >= query_lens[b]`` give
    zeros.  ``window`` (a sliding-window layer): of the prefix only the last
    ``window`` keys are visible (gqa_attention.py:305-314); with ``k_draft``
    / ``v_draft`` (fp16 ``[B, S, Hkv, D]``, the layer's fresh draft K / V)
    the drafts are attended with those values, as the reference's window
    verify concatenates them to the dequantized prefix window
    (gqa_attention.py:298-303).  Returns fp16 ``[B, Hq, S, D]``."""
    keep, head, tail, workspace, (n, hkv, bs, d), out = _verify_inputs(
        q, k_cache, k_scale, block_table, prefix_lens, block_size, query_lens, tree_mask, max_context_len)
    dev = out.device
    _on_gpu("v_cache", v_cache, torch.int8, dev)
    _on_gpu("v_scale", v_scale, torch.float32, dev)
    _require(v_cache.shape == k_cache.shape and v_cache.is_contiguous(), "v_cache must match k_cache")
    _require(tuple(v_scale.shape) == (n, hkv, bs) and v_scale.is_contiguous(), "v_scale must be [N, Hkv, bs]")
    if out.shape[0] == 0 or out.shape[2] == 0:
        return out
    lib = _lib.load()
    _require(window is not None or k_draft is None, "fresh drafts (k_draft / v_draft) need a window")
    if window is not None:
        _require(int(window) >= 1, f"window must be >= 1, got {window}")
        alive, drafts = _fresh_drafts(k_draft, v_draft, out.shape[0], out.shape[2], hkv, d, dev)
        rc = lib.s8kv_verify_window_int8(
            *head, k_cache.data_ptr(), k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(), n, bs,
            *tail, int(window), *drafts, float(scale), out.data_ptr(), *workspace, _stream(keep[0]),
        )
    else:
        rc = lib.s8kv_verify_int8(
            *head, k_cache.data_ptr(), k_scale.data_ptr(), v_cache.data_ptr(), v_scale.data_ptr(), n, bs,
            *tail, float(scale), out.data_ptr(), *workspace, _stream(keep[0]),
        )
    _lib.check(rc, "attn_paged_verify")
    return out


def attn_paged_verify_k8v3(q, k_cache, k_scale, v_packed, v_norm, v_codebook, block_table, prefix_lens, block_size,
                           *, query_lens=None, tree_mask=None, max_context_len, scale, window=None, k_draft=None,
                           v_draft=None):
    """``attn_paged_verify`` over the K8V3 cache (int8 K, 3-bit Lloyd-Max V
    ``codebook[code] * block norm``): one launch for what the reference
    computes on a k8v3 cache with S sequential ``attn_paged_decode_k8v3``
    calls (chain verify, gqa_attention.py:259-277) or ``read_dense`` plus
    dense attention (chunked prefill).  head_dim 128 or 256, lloyd_block 128."""
    keep, head, tail, workspace, (n, hkv, bs, d), out = _verify_inputs(
        q, k_cache, k_scale, block_table, prefix_lens, block_size, query_lens, tree_mask, max_context_len)
    dev = out.device
    _on_gpu("v_packed", v_packed, torch.int32, dev)
    _on_gpu("v_norm", v_norm, torch.float32, dev)
    _on_gpu("v_codebook", v_codebook, torch.float32, dev)
    _require(tuple(v_packed.shape) == (n, hkv, bs, d * 3 // 32) and v_packed.is_contiguous(),
             "v_packed must be [N, Hkv, bs, D*3/32]")
    lloyd_block = d // v_norm.shape[-1] if v_norm.dim() == 4 and v_norm.shape[-1] > 0 else 0
    _require(tuple(v_norm.shape[:3]) == (n, hkv, bs) and v_norm.is_contiguous(), "v_norm must be [N, Hkv, bs, D/128]")
    _require(v_codebook.numel() == 8 and v_codebook.is_contiguous(), "v_codebook must hold 8 contiguous entries")
    if out.shape[0] == 0 or out.shape[2] == 0:
        return out
    lib = _lib.load()
    _require(window is not None or k_draft is None, "fresh drafts (k_draft / v_draft) need a window")
    if window is not None:
        _require(int(window) >= 1, f"window must be >= 1, got {window}")
        alive, drafts = _fresh_drafts(k_draft, v_draft, out.shape[0], out.shape[2], hkv, d, dev)
        rc = lib.s8kv_verify_window_k8v3(
            *head, k_cache.data_ptr(), k_scale.data_ptr(), v_packed.data_ptr(), v_norm.data_ptr(),
            v_codebook.data_ptr(), lloyd_block, n, bs, *tail, int(window), *drafts, float(scale), out.data_ptr(),
            *workspace, _stream(keep[0]),
        )
    else:
        rc = lib.s8kv_verify_k8v3(
            *head, k_cache.data_ptr(), k_scale.data_ptr(), v_packed.data_ptr(), v_norm.data_ptr(),
            v_codebook.data_ptr(), lloyd_block, n, bs, *tail, float(scale), out.data_ptr(), *workspace,
            _stream(keep[0]),
        )
    _lib.check(rc, "attn_paged_verify_k8v3")
    return out


def attn_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, *, causal, scale, window_left=None):
    """Prefill attention over fresh fp16 K / V, varlen batched (the role of
    ``superl8.attn_int8_varlen``, gqa_attention.py:81-104): ``q`` fp16
    ``[Tq, Hq, D]``, ``k``, ``v`` fp16 ``[Tk, Hkv, D]`` token-major (head_dim
    contiguous), sequences delimited by int32 ``cu_seqlens_q`` / ``cu_seqlens_k``
    (``[B + 1]``).  ``causal``: bottom-right aligned.  ``window_left >= 1``
    (causal only): query i sees only its last ``window_left`` keys, itself
    included -- the keys the reference's sliding-window decode attends for
    the same layer (gqa_attention.py:150-154).  Returns fp16 ``[Tq, Hq, D]``."""
    _on_gpu("q", q, torch.float16)
    dev = q.device
    _on_gpu("k", k, torch.float16, dev)
    _on_gpu("v", v, torch.float16, dev)
    _on_gpu("cu_seqlens_q", cu_seqlens_q, torch.int32, dev)
    _on_gpu("cu_seqlens_k", cu_seqlens_k, torch.int32, dev)
    _require(q.dim() == 3 and k.dim() == 3 and v.shape == k.shape and k.shape[2] == q.shape[2],
             "attn_varlen: q [Tq, Hq, D], k / v [Tk, Hkv, D]")
    _require(window_left is None or int(window_left) >= 1, f"window_left must be >= 1, got {window_left}")
    tq, hq, d = q.shape
    hkv = k.shape[1]
    _require(cu_seqlens_q.dim() == 1 and cu_seqlens_q.shape == cu_seqlens_k.shape and cu_seqlens_q.numel() >= 1,
             "attn_varlen: cu_seqlens_q / cu_seqlens_k must be [B + 1]")
    if q.stride(2) != 1:
        q = q.contiguous()
    if k.stride(2) != 1 or k.data_ptr() % 16 or k.stride(0) % 8 or k.stride(1) % 8:
        k = k.contiguous()
    if v.stride(2) != 1 or v.data_ptr() % 16 or v.stride(0) % 8 or v.stride(1) % 8:
        v = v.contiguous()
    cu_q, cu_k = cu_seqlens_q.contiguous(), cu_seqlens_k.contiguous()
    out = torch.zeros((tq, hq, d), dtype=torch.float16, device=dev)
    b = cu_q.numel() - 1
    if b == 0 or tq == 0:
        return out
    lib = _lib.load()
    rc = lib.s8kv_attn_varlen_f16(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), cu_q.data_ptr(), cu_k.data_ptr(), b, hq, hkv, d,
        int(max_seqlen_q), int(max_seqlen_k), q.stride(0), q.stride(1), k.stride(0), k.stride(1), v.stride(0),
        v.stride(1), 1 if causal else 0, -1 if window_left is None else int(window_left), float(scale),
        out.data_ptr(), out.stride(0), out.stride(1), _stream(q),
    )
    _lib.check(rc, "attn_varlen")
    return out


def attn_fwd(q, k, v, *, causal, scale, window_left=None):
    """Dense prefill attention over fresh fp16 K / V in the ``[B, H, S, D]``
    layout (the role of ``superl8.attn_int8_fwd`` on fresh K / V,
    gqa_attention.py:124-128): ``q`` ``[B, Hq, Sq, D]``, ``k``, ``v``
    ``[B, Hkv, Sk, D]``; causal is bottom-right aligned; ``window_left`` as
    in ``attn_varlen`` (negative: none).  Runs
    ``attn_varlen`` on token-major copies.  Returns fp16 ``[B, Hq, Sq, D]``."""
    _require(q.dim() == 4 and k.dim() == 4 and v.shape == k.shape, "attn_fwd: q [B, Hq, Sq, D], k / v [B, Hkv, Sk, D]")
    b, hq, sq, d = q.shape
    sk = k.shape[2]
    qt = q.transpose(1, 2).reshape(b * sq, hq, d)
    kt = k.transpose(1, 2).reshape(b * sk, k.shape[1], d)
    vt = v.transpose(1, 2).reshape(b * sk, v.shape[1], d)
    cu_q = torch.arange(0, (b + 1) * sq, sq, dtype=torch.int32, device=q.device)
    cu_k = torch.arange(0, (b + 1) * sk, sk, dtype=torch.int32, device=q.device)
    out = attn_varlen(qt, kt, vt, cu_q, cu_k, sq, sk, causal=causal, scale=scale,
                      window_left=None if window_left is None or window_left < 0 else window_left)
    return out.reshape(b, sq, hq, d).transpose(1, 2)


def copy_blocks(tensors: Sequence[torch.Tensor], src: Sequence[int] | torch.Tensor,
                dst: Sequence[int] | torch.Tensor) -> None:
    """Byte copy ``t[:, dst[i]] = t[:, src[i]]`` for every cache tensor
    ``t`` laid out ``[num_layers, num_blocks, ...]`` (copy-on-write and pool
    compaction).  ``src``/``dst`` are host integer sequences (validated here:
    in range, equal length, disjoint) or int32 device tensors."""
    _require(1 <= len(tensors) <= 8, "copy_blocks takes 1..8 tensors")
    t0 = tensors[0]
    _on_gpu("tensors[0]", t0)
    dev = t0.device
    nl, nb = t0.shape[0], t0.shape[1]
    ptrs, bbytes, lstrides = [], [], []
    for i, t in enumerate(tensors):
        _on_gpu(f"tensors[{i}]", t, None, dev)
        _require(t.is_contiguous(), f"tensors[{i}] must be contiguous")
        _require(t.shape[0] == nl and t.shape[1] == nb, f"tensors[{i}] must be [{nl}, {nb}, ...]")
        per_block = t[0, 0].numel() * t.element_size()
        ptrs.append(t.data_ptr())
        bbytes.append(per_block)
        lstrides.append(t.stride(0) * t.element_size())
    if isinstance(src, torch.Tensor) or isinstance(dst, torch.Tensor):
        _require(isinstance(src, torch.Tensor) and isinstance(dst, torch.Tensor), "src and dst must both be tensors")
        _on_gpu("src", src, torch.int32, dev)
        _on_gpu("dst", dst, torch.int32, dev)
        src_t, dst_t = src.contiguous(), dst.contiguous()
        _require(src_t.numel() == dst_t.numel(), "src and dst differ in length")
    else:
        src_l, dst_l = [int(x) for x in src], [int(x) for x in dst]
        _require(len(src_l) == len(dst_l), "src and dst differ in length")
        _require(all(0 <= x < nb for x in src_l + dst_l), f"block ids must be in [0, {nb})")
        _require(not (set(src_l) & set(dst_l)), "source and destination blocks overlap")
        _require(len(set(dst_l)) == len(dst_l), "destination blocks repeat")
        if not src_l:
            return
        src_t = torch.tensor(src_l, dtype=torch.int32).to(dev, non_blocking=True)
        dst_t = torch.tensor(dst_l, dtype=torch.int32).to(dev, non_blocking=True)
    npairs = src_t.numel()
    if npairs == 0:
        return
    n = len(tensors)
    arr_p = (ctypes.c_void_p * n)(*ptrs)
    arr_b = (ctypes.c_int64 * n)(*bbytes)
    arr_s = (ctypes.c_int64 * n)(*lstrides)
    rc = _lib.load().s8kv_copy_blocks(n, arr_p, arr_b, arr_s, nl, nb, src_t.data_ptr(), dst_t.data_ptr(), npairs,
                                      _stream(t0))
    _lib.check(rc, "copy_blocks")


# ---------------------------------------------------------------------------
# Row codecs (the helpers the reference's cache code calls on ``superl8``)
# ---------------------------------------------------------------------------

_ROT_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def _rows_view(x: torch.Tensor, name: str) -> torch.Tensor:
    """``x`` as ``[rows, D]`` with a unit stride on D (copies when the leading
    axes cannot be flattened into one row stride)."""
    _require(x.dim() >= 1, f"{name} must have at least one dimension")
    d = x.shape[-1]
    x2 = x.reshape(-1, d)
    if x2.numel() and (x2.stride(1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < d)):
        x2 = x2.contiguous()
    return x2


def rotate_rows(x: torch.Tensor) -> torch.Tensor:
    """``rotate_last``: the normalized Hadamard rotation of the last axis
    (fp32 transform, one multiply by fp32(1/sqrt(D)), one rounding to x's
    dtype), the rotation the append applies to K.  fp16, bf16 or fp32; D in
    {32, 64, 128, 256}.  Returns a new tensor of x's shape and dtype."""
    _on_gpu("x", x)
    _require(x.dtype in _ROT_DTYPES, f"rotate_last: dtype {x.dtype} not in fp16 / bf16 / fp32", TypeError)
    x2 = _rows_view(x, "x")
    d = x.shape[-1]
    out = torch.empty(x2.shape, dtype=x.dtype, device=x.device)
    if x2.shape[0]:
        lib = _lib.load()
        rc = lib.s8kv_rotate_rows(x2.data_ptr(), x2.shape[0], d, x2.stride(0), _ROT_DTYPES[x.dtype], out.data_ptr(),
                                  out.stride(0), _stream(x))
        _lib.check(rc, "rotate_last")
    return out.reshape(x.shape)


def quantize_rows_int8(x: torch.Tensor, rotate: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row symmetric RTN int8 of fp16 rows (``quantize_i8_rowwise``):
    int8 codes of x's shape and fp32 scales ``x.shape[:-1]``; ``rotate``
    applies ``rotate_last`` first, in the same pass (the append's K bytes)."""
    _on_gpu("x", x, torch.float16)
    x2 = _rows_view(x, "x")
    d = x.shape[-1]
    q = torch.empty(x2.shape, dtype=torch.int8, device=x.device)
    sc = torch.empty(x2.shape[0], dtype=torch.float32, device=x.device)
    if x2.shape[0]:
        lib = _lib.load()
        rc = lib.s8kv_quantize_rows_int8(x2.data_ptr(), x2.shape[0], d, x2.stride(0), 1 if rotate else 0,
                                         q.data_ptr(), sc.data_ptr(), _stream(x))
        _lib.check(rc, "quantize_i8_rowwise")
    return q.reshape(x.shape), sc.reshape(x.shape[:-1])


def quantize_rows_lloydmax3(v: torch.Tensor, codebook: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """3-bit Lloyd-Max codes (uint8, v's shape) and per-128 block norms (fp32,
    ``v.shape[:-1] + (D/128,)``) of fp16 rows -- the append's K8V3 V path."""
    _on_gpu("v", v, torch.float16)
    dev = v.device
    _on_gpu("codebook", codebook, torch.float32, dev)
    _require(codebook.numel() == 8, "codebook must hold 8 entries")
    cb = codebook.reshape(8).contiguous()
    v2 = _rows_view(v, "v")
    d = v.shape[-1]
    codes = torch.empty(v2.shape, dtype=torch.uint8, device=dev)
    norms = torch.empty((v2.shape[0], max(1, d // 128)), dtype=torch.float32, device=dev)
    if v2.shape[0]:
        lib = _lib.load()
        rc = lib.s8kv_quantize_rows_lloydmax3(v2.data_ptr(), v2.shape[0], d, v2.stride(0), cb.data_ptr(),
                                              codes.data_ptr(), norms.data_ptr(), _stream(v))
        _lib.check(rc, "quantize_lloydmax")
    return codes.reshape(v.shape), norms.reshape(*v.shape[:-1], -1)


def pack_codes3(codes: torch.Tensor) -> torch.Tensor:
    """Bit-plane words (int32, ``[..., 3D/32]``) of uint8 3-bit codes
    ``[..., D]``: word 3g+b holds bit b of codes 32g..32g+31 (the cache's
    ``v_packed`` layout)."""
    _on_gpu("codes", codes, torch.uint8)
    c2 = codes.reshape(-1, codes.shape[-1]).contiguous()
    d = codes.shape[-1]
    _require(d % 32 == 0, f"pack_indices_lowbit: last dimension {d} is not a multiple of 32")
    words = torch.empty((c2.shape[0], d * 3 // 32), dtype=torch.int32, device=codes.device)
    if c2.numel():
        lib = _lib.load()
        _lib.check(lib.s8kv_pack_codes3(c2.data_ptr(), c2.shape[0], d, words.data_ptr(), _stream(codes)),
                   "pack_indices_lowbit")
    return words.reshape(*codes.shape[:-1], d * 3 // 32)


def unpack_codes3(words: torch.Tensor, d: int) -> torch.Tensor:
    """Inverse of ``pack_codes3``: int32 words ``[..., 3d/32]`` -> uint8 codes
    ``[..., d]``."""
    _on_gpu("words", words, torch.int32)
    d = int(d)
    _require(d > 0 and d % 32 == 0 and words.shape[-1] == d * 3 // 32,
             f"unpack_indices_lowbit: {words.shape[-1]} words per row do not hold {d} 3-bit codes")
    w2 = words.reshape(-1, words.shape[-1]).contiguous()
    codes = torch.empty((w2.shape[0], d), dtype=torch.uint8, device=words.device)
    if w2.numel():
        lib = _lib.load()
        _lib.check(lib.s8kv_unpack_codes3(w2.data_ptr(), w2.shape[0], d, codes.data_ptr(), _stream(words)),
                   "unpack_indices_lowbit")
    return codes.reshape(*words.shape[:-1], d)


# ---------------------------------------------------------------------------
# Prompt-time eviction: SnapKV scores and the keep-list gather
# ---------------------------------------------------------------------------


def _q_rows(q: torch.Tensor, num_q_heads: int) -> torch.Tensor:
    _require(q.dtype in (torch.float16, torch.float32), f"q must be fp16 or fp32, got {q.dtype}", TypeError)
    q2 = q.reshape(num_q_heads, -1)
    if q2.stride(1) != 1:
        q2 = q2.contiguous()
    return q2


def _snapkv_run(n: int, hq: int, dev, launch) -> torch.Tensor:
    scores = torch.empty(n, dtype=torch.float32, device=dev)
    if n == 0:
        return scores
    lib = _lib.load()
    ws_bytes = int(lib.s8kv_snapkv_workspace_size(hq, n))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    _lib.check(launch(lib, scores, ws, ws_bytes), "snapkv_scores")
    return scores


def snapkv_scores(q: torch.Tensor, k: torch.Tensor, num_heads: int, num_kv_heads: int, scale: float | None = None
                  ) -> torch.Tensor:
    """SnapKV scores over a dense K (``KVEviction.snapkv_selection``'s
    ranking, kv_cache.py:149-163): ``q`` ``[num_heads, D]`` (any shape with
    that many elements), ``k`` ``[Hkv, S, D]`` or ``[1, Hkv, S, D]``, fp16 or
    fp32; returns fp32 ``[S]``, the mean over q heads of
    ``softmax(q_h . k / sqrt(D))`` (``scale`` overrides 1/sqrt(D))."""
    _on_gpu("q_last", q)
    _on_gpu("k_full", k, None, q.device)
    if k.dim() == 4:
        _require(k.shape[0] == 1, "k_full [1, Hkv, S, D] expected")
        k = k[0]
    _require(k.dim() == 3 and k.shape[0] == num_kv_heads, f"k_full must be [{num_kv_heads}, S, D]")
    _require(k.dtype in (torch.float16, torch.float32), f"k_full must be fp16 or fp32, got {k.dtype}", TypeError)
    d = k.shape[2]
    q2 = _q_rows(q, num_heads)
    _require(q2.shape[1] == d, f"q_last head_dim {q2.shape[1]} != k_full head_dim {d}")
    if k.stride(2) != 1:
        k = k.contiguous()
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    return _snapkv_run(k.shape[1], num_heads, q.device, lambda lib, out, ws, nb: lib.s8kv_snapkv_scores_dense(
        q2.data_ptr(), 1 if q2.dtype == torch.float32 else 0, q2.stride(0), num_heads, num_kv_heads, d, k.data_ptr(),
        1 if k.dtype == torch.float32 else 0, k.stride(0), k.stride(1), k.shape[1], sc, out.data_ptr(), ws.data_ptr(),
        nb, _stream(q2)))


def snapkv_scores_paged(q: torch.Tensor, k_cache: torch.Tensor, k_scale: torch.Tensor, blocks: Sequence[int],
                        length: int, num_heads: int, scale: float | None = None) -> torch.Tensor:
    """SnapKV scores of one sequence over its int8 K in the paged cache
    (``k_cache`` ``[N, Hkv, bs, D]`` layer view, ``blocks`` its block ids in
    order): the same quantity as ``snapkv_scores`` over the exactly
    dequantized keys, without materializing them."""
    _on_gpu("q_last", q)
    dev = q.device
    _on_gpu("k_cache", k_cache, torch.int8, dev)
    _on_gpu("k_scale", k_scale, torch.float32, dev)
    n, hkv, bs, d = _cache_geometry(k_cache)
    _require(tuple(k_scale.shape) == (n, hkv, bs) and k_scale.is_contiguous(), "k_scale must be [N, Hkv, bs]")
    length = int(length)
    need = -(-length // bs)
    blocks = [int(b) for b in blocks]
    _require(len(blocks) >= need, f"{len(blocks)} blocks cannot hold {length} tokens")
    _require(all(0 <= b < n for b in blocks[:need]), f"block ids must be in [0, {n})")
    q2 = _q_rows(q, num_heads)
    _require(q2.shape[1] == d, f"q_last head_dim {q2.shape[1]} != cache head_dim {d}")
    row = torch.tensor(blocks[:max(need, 1)], dtype=torch.int32).to(dev)
    sc = 1.0 / math.sqrt(d) if scale is None else float(scale)
    return _snapkv_run(length, num_heads, dev, lambda lib, out, ws, nb: lib.s8kv_snapkv_scores_paged(
        q2.data_ptr(), 1 if q2.dtype == torch.float32 else 0, q2.stride(0), num_heads, hkv, d, k_cache.data_ptr(),
        k_scale.data_ptr(), n, bs, row.data_ptr(), length, sc, out.data_ptr(), ws.data_ptr(), nb, _stream(q2)))


def gather_slots(tensors: Sequence[torch.Tensor], src_slots: Sequence[int], dst_slots: Sequence[int],
                 block_size: int) -> None:
    """Copy the rows of flat slots ``src_slots[j]`` to ``dst_slots[j]`` in
    every layer of every cache tensor (``[L, N, Hkv, bs, ...]``), byte for
    byte: the kept tokens of a keep-list compaction."""
    _require(1 <= len(tensors) <= 8, "gather_slots takes 1..8 tensors")
    src_l, dst_l = [int(x) for x in src_slots], [int(x) for x in dst_slots]
    _require(len(src_l) == len(dst_l), "src and dst differ in length")
    if not src_l:
        return
    t0 = tensors[0]
    _on_gpu("tensors[0]", t0)
    dev = t0.device
    nl, nb, hkv, bs = t0.shape[:4]
    _require(int(block_size) == bs, f"block_size {block_size} does not match the cache ({bs})")
    _require(all(0 <= x < nb * bs for x in src_l + dst_l), f"slots must be in [0, {nb * bs})")
    _require(not (set(src_l) & set(dst_l)), "source and destination slots overlap")
    ptrs, rbytes, lstrides = [], [], []
    for i, t in enumerate(tensors):
        _on_gpu(f"tensors[{i}]", t, None, dev)
        _require(t.is_contiguous() and tuple(t.shape[:4]) == (nl, nb, hkv, bs),
                 f"tensors[{i}] must be contiguous [{nl}, {nb}, {hkv}, {bs}, ...]")
        ptrs.append(t.data_ptr())
        rbytes.append(t[0, 0, 0, 0].numel() * t.element_size())
        lstrides.append(t.stride(0) * t.element_size())
    src_t = torch.tensor(src_l, dtype=torch.int32).to(dev)
    dst_t = torch.tensor(dst_l, dtype=torch.int32).to(dev)
    n = len(tensors)
    rc = _lib.load().s8kv_gather_slots(n, (ctypes.c_void_p * n)(*ptrs), (ctypes.c_int64 * n)(*rbytes),
                                       (ctypes.c_int64 * n)(*lstrides), nl, hkv, nb, bs, src_t.data_ptr(),
                                       dst_t.data_ptr(), len(src_l), _stream(t0))
    _lib.check(rc, "gather_slots")
