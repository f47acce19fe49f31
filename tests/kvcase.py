"""Seeded paged-KV test cases shared by the CPU and GPU tests.

A case is a pool of physical blocks, a fragmented block table and per-row
context lengths; caches are filled through the oracle's append so the GPU
kernels can be compared with it byte for byte."""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from oracle import kv_oracle as O


@dataclass
class PagedCase:
    batch: int
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    lens: np.ndarray  # int context lengths (after the append)
    num_blocks: int
    block_table: np.ndarray  # int32 [B, W]
    k: np.ndarray = field(default=None)  # fp16 [sum L, Hkv, D] per-token K (token-major, row by row)
    v: np.ndarray = field(default=None)
    slots: np.ndarray = field(default=None)  # int32 flat slot of every token in k/v order
    q: np.ndarray = field(default=None)  # fp16 [B, Hq, D]

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)


def make_case(seed: int, batch: int, hq: int, hkv: int, d: int, bs: int, lens, *, spare_blocks: int = 4,
              outlier_channels: int = 0, outlier_scale: float = 20.0, width: int | None = None) -> PagedCase:
    """Random case: blocks dealt from a seeded permutation of the pool, K/V/q
    ~N(0,1) fp16 with optional outlier channels scaled by `outlier_scale`."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    need = [(int(n) + bs - 1) // bs for n in lens]
    n_blocks = sum(need) + spare_blocks
    perm = rng.permutation(n_blocks)
    w = width if width is not None else max(1, max(need) if need else 1)
    bt = np.zeros((batch, w), dtype=np.int32)
    pos = 0
    for b in range(batch):
        bt[b, : need[b]] = perm[pos: pos + need[b]]
        pos += need[b]
    total = int(lens.sum())
    k = rng.standard_normal((total, hkv, d)).astype(np.float32)
    v = rng.standard_normal((total, hkv, d)).astype(np.float32)
    q = rng.standard_normal((batch, hq, d)).astype(np.float32)
    if outlier_channels:
        ch = rng.choice(d, size=outlier_channels, replace=False)
        k[..., ch] *= outlier_scale
        v[..., ch] *= outlier_scale
        q[..., ch] *= outlier_scale
    slots = np.zeros(total, dtype=np.int32)
    i = 0
    for b in range(batch):
        for p in range(int(lens[b])):
            slots[i] = bt[b, p // bs] * bs + p % bs
            i += 1
    return PagedCase(batch, hq, hkv, d, bs, lens, n_blocks, bt, k.astype(np.float16), v.astype(np.float16), slots,
                     q.astype(np.float16))


def empty_int8_cache(case: PagedCase):
    shape = (case.num_blocks, case.num_kv_heads, case.block_size, case.head_dim)
    return (np.zeros(shape, np.int8), np.ones(shape[:3], np.float32), np.zeros(shape, np.int8),
            np.ones(shape[:3], np.float32))


def empty_k8v3_cache(case: PagedCase):
    shape = (case.num_blocks, case.num_kv_heads, case.block_size, case.head_dim)
    d = case.head_dim
    return (np.zeros(shape, np.int8), np.ones(shape[:3], np.float32),
            np.zeros(shape[:3] + (d * 3 // 32,), np.int32), np.zeros(shape[:3] + (d // 128,), np.float32))


def oracle_fill_int8(case: PagedCase):
    kc, ks, vc, vs = empty_int8_cache(case)
    O.quantize_kv_write_paged(case.k, case.v, kc, ks, vc, vs, case.slots)
    return kc, ks, vc, vs


def oracle_fill_k8v3(case: PagedCase, codebook):
    kc, ks, vp, vn = empty_k8v3_cache(case)
    O.k8v3_write_paged(case.k, case.v, kc, ks, vp, vn, codebook, case.slots)
    return kc, ks, vp, vn
