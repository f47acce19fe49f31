"""PyTorch-CPU restatement of the reference's host path for append + decode.

TEST INFRASTRUCTURE ONLY (the ``cpu_baseline`` leg of ``bench.py`` and the
tests).  It follows the structure of the reference's own CPU-capable code:

* append: ``_flat_rows`` scatter (kv_cache.py:570-585) of ``rotate_last``
  (``(x.float() @ H).to(fp16)``, dist/pipeline.py:51-59) followed by the
  per-row RTN of ``quantize_i8_rowwise`` (kv_cache.py:587-604);
* decode: per-slot ``read_dense`` (kv_cache.py:1233-1299) and an fp32 softmax
  attention per sequence -- the shape of the reference's per-slot fallback
  (kv_cache.py:673-689, gqa_attention.py:191-196).

Everything runs with torch's intra-op thread pool (``torch.set_num_threads``).
"""

from __future__ import annotations

import math

import torch


def hadamard(d: int, dtype=torch.float32) -> torch.Tensor:
    h = torch.ones(1, 1, dtype=torch.float64)
    while h.shape[0] < d:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    return (h / math.sqrt(d)).to(dtype)


def rotate_last(x: torch.Tensor, h: torch.Tensor) -> torch.Tensor:
    return (x.float() @ h).to(x.dtype)


def quantize_rows(x: torch.Tensor):
    xf = x.float()
    s = xf.abs().amax(-1) / 127.0
    q = torch.where(s[..., None] > 0, torch.round(xf / torch.where(s > 0, s, 1.0)[..., None]), 0.0)
    return q.clamp_(-127, 127).to(torch.int8), s


def flat_rows(slot_mapping: torch.Tensor, hkv: int, bs: int) -> torch.Tensor:
    blk = slot_mapping.long() // bs
    off = slot_mapping.long() % bs
    heads = torch.arange(hkv)
    return ((blk[:, None] * hkv + heads[None]) * bs + off[:, None]).reshape(-1)


def append(k, v, k_cache, k_scale, v_cache, v_scale, slot_mapping, h) -> None:
    """k, v: fp16 [T, Hkv, D]; caches: per-layer views [N, Hkv, bs, D]."""
    t, hkv, d = k.shape
    bs = k_cache.shape[2]
    kq, ks = quantize_rows(rotate_last(k, h).reshape(-1, d))
    vq, vs = quantize_rows(v.reshape(-1, d))
    rows = flat_rows(slot_mapping, hkv, bs)
    k_cache.view(-1, d)[rows] = kq
    k_scale.view(-1)[rows] = ks
    v_cache.view(-1, d)[rows] = vq
    v_scale.view(-1)[rows] = vs


def read_dense(k_cache, k_scale, v_cache, v_scale, blocks: list[int], length: int, h):
    """Dequantized fp16 K, V ``[Hkv, n, D]`` of one sequence (kv_cache.py:1286-1298)."""
    bs = k_cache.shape[2]
    pos = torch.arange(length)
    blk = torch.tensor(blocks, dtype=torch.long)[pos // bs]
    off = pos % bs
    k = (k_cache[blk, :, off, :].float() * k_scale[blk, :, off].unsqueeze(-1)).half()
    v = (v_cache[blk, :, off, :].float() * v_scale[blk, :, off].unsqueeze(-1)).half()
    return rotate_last(k, h).permute(1, 0, 2), v.permute(1, 0, 2)


def decode(q, k_cache, k_scale, v_cache, v_scale, block_lists: list[list[int]], lens: list[int], scale: float, h):
    """q: fp16 [B, Hq, D] -> fp32 [B, Hq, D]; per-slot dense dequant + fp32 attention."""
    b_, hq, d = q.shape
    hkv = k_cache.shape[1]
    g = hq // hkv
    out = torch.empty(b_, hq, d, dtype=torch.float32)
    for b in range(b_):
        k, v = read_dense(k_cache, k_scale, v_cache, v_scale, block_lists[b], int(lens[b]), h)
        qb = q[b].float().view(hkv, g, d)
        s = torch.bmm(qb, k.float().transpose(1, 2)) * scale
        p = torch.softmax(s, dim=-1)
        out[b] = torch.bmm(p, v.float()).reshape(hq, d)
    return out
