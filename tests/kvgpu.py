"""GPU-side helpers shared by the GPU tests: cache allocation and the ops of
either cache layout (int8, or K8V3: int8 K with 3-bit Lloyd-Max V) behind one
call each."""

from __future__ import annotations

import numpy as np
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops

DEV = "cuda"
CODEBOOK = O.gaussian_codebook(3, 128)
KINDS = ("int8", "k8v3")


def t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def to_np(x):
    return x.detach().cpu().numpy()


def alloc(kind, n, hkv, bs, d):
    """An empty cache of ``n`` blocks (the oracle's empty-cache values)."""
    shape = (n, hkv, bs, d)
    kc = torch.zeros(shape, dtype=torch.int8, device=DEV)
    ks = torch.ones(shape[:3], dtype=torch.float32, device=DEV)
    if kind == "int8":
        return (kc, ks, torch.zeros(shape, dtype=torch.int8, device=DEV),
                torch.ones(shape[:3], dtype=torch.float32, device=DEV))
    return (kc, ks, torch.zeros(shape[:3] + (d * 3 // 32,), dtype=torch.int32, device=DEV),
            torch.zeros(shape[:3] + (d // 128,), dtype=torch.float32, device=DEV))


def _codebook(kind):
    return () if kind == "int8" else (t(CODEBOOK),)


def append(kind, k, v, cache, slots):
    if kind == "int8":
        ops.quantize_kv_write_paged(k, v, *cache, slots)
    else:
        ops.quantize_kv_write_paged_k8v3(k, v, *cache, t(CODEBOOK), slots)


def decode(kind, q, cache, bt, lens, bs, max_ctx, scale):
    fn = ops.attn_paged_decode_cached if kind == "int8" else ops.attn_paged_decode_k8v3
    return fn(q, *cache, *_codebook(kind), bt, lens, bs, max_context_len=max_ctx, scale=scale)


def decode_append(kind, q, k_new, v_new, cache, bt, lens, bs, max_ctx, scale, plan=None):
    fn = ops.attn_paged_decode_append if kind == "int8" else ops.attn_paged_decode_append_k8v3
    return fn(q, k_new, v_new, *cache, *_codebook(kind), bt, lens, bs, max_context_len=max_ctx, scale=scale,
              plan=plan)


def decode_plan(kind, cache, bt, lens, bs, hq, max_ctx):
    return ops.attn_paged_decode_plan(cache[0], bt, lens, bs, num_q_heads=hq, max_context_len=max_ctx,
                                      layout="int8" if kind == "int8" else "k8v3")


def verify(kind, q, cache, bt, prefix, query_lens, bs, max_ctx, scale):
    fn = ops.attn_paged_verify if kind == "int8" else ops.attn_paged_verify_k8v3
    return fn(q, *cache, *_codebook(kind), bt, prefix, bs, query_lens=query_lens, max_context_len=max_ctx,
              scale=scale)


def layer(kind, cache):
    """The oracle's view of a (numpy) cache."""
    if kind == "int8":
        return O.LayerCache(*cache)
    kc, ks, vp, vn = cache
    return O.LayerCache(kc, ks, v_packed=vp, v_norm=vn, v_codebook=CODEBOOK)


def assert_close(out, ref, what):
    mx, rel = O.attention_errors(out, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"
