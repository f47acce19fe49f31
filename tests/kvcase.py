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


@dataclass
class NeedleCase:
    """One sequence through every block of an Hkv-1 pool: zero keys (score 0)
    with one constant V row ``u_i8 / 128`` everywhere but one needle token
    per q head.  q head h is a multiple of Hadamard row ``chans[h]``, so it
    scores its own needle (K row ``127 e_chans[h]``) near ``ln(n)`` and the
    other needles 0."""
    block_size: int
    head_dim: int
    block_table: np.ndarray  # int32 [nblk]: a shuffle whose last entry is the pool's last block
    pos: np.ndarray  # int64 [Hq] needle positions in the sequence (needle 0: the last position)
    rows: np.ndarray  # int64 [Hq] their flat cache rows
    k_i8: np.ndarray  # int8 [Hq, D] needle K rows (as stored: rotated, quantized)
    k_scale: np.ndarray  # float32 [Hq]
    v_i8: np.ndarray  # int8 [Hq, D]
    v_scale: np.ndarray  # float32 [Hq]
    u_i8: np.ndarray  # int8 [D] background V row (scale 1/128; background K scale 1/128)
    q: np.ndarray  # fp16 [Hq, D]

    @property
    def n(self) -> int:
        return len(self.block_table) * self.block_size

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)


def make_needle_case(seed: int, nblk: int, bs: int, d: int, hq: int, marks) -> NeedleCase:
    """Needle 0 at the sequence's last position, which the table puts in the
    pool's last row; needles 1.. at ``(block, offset)`` of ``marks``, then
    the sequence's first position, then random positions."""
    rng = np.random.default_rng(seed)
    bt = rng.permutation(nblk).astype(np.int32)
    top = int(np.nonzero(bt == nblk - 1)[0][0])
    bt[[top, nblk - 1]] = bt[[nblk - 1, top]]
    where = np.empty(nblk, np.int64)
    where[bt] = np.arange(nblk)
    n = nblk * bs
    pos = [n - 1] + [int(where[blk]) * bs + off for blk, off in marks] + [0]
    while len(pos) < hq:
        p = int(rng.integers(1, n - 1))
        if p not in pos:
            pos.append(p)
    pos = np.array(pos[:hq], np.int64)
    if len(set(pos.tolist())) != hq:
        raise ValueError("needle positions collide")
    rows = bt[pos // bs].astype(np.int64) * bs + pos % bs
    chans = rng.choice(d, size=hq, replace=False)
    k_i8 = np.zeros((hq, d), np.int8)
    k_i8[np.arange(hq), chans] = 127
    k_scale = np.full(hq, 0.11, np.float32)
    scale = 1.0 / math.sqrt(d)
    target = math.log(n) + rng.uniform(-1.5, 1.5, size=hq)
    q = ((target / (scale * 127 * float(k_scale[0])))[:, None] * O.hadamard_matrix(d)[chans]).astype(np.float16)
    return NeedleCase(bs, d, bt, pos, rows, k_i8, k_scale, rng.integers(-127, 128, size=(hq, d)).astype(np.int8),
                      rng.uniform(1 / 128, 1 / 32, size=hq).astype(np.float32),
                      rng.integers(-100, 101, size=d).astype(np.int8), q)


def needle_fill(nc: NeedleCase):
    """The case's int8 cache ``(k, k_scale, v, v_scale)`` in numpy (small pools)."""
    nblk, bs, d = len(nc.block_table), nc.block_size, nc.head_dim
    kc = np.zeros((nblk, 1, bs, d), np.int8)
    ks = np.full((nblk, 1, bs), 1 / 128, np.float32)
    vc = np.broadcast_to(nc.u_i8, (nblk, 1, bs, d)).copy()
    vs = np.full((nblk, 1, bs), 1 / 128, np.float32)
    kc.reshape(-1, d)[nc.rows] = nc.k_i8
    ks.reshape(-1)[nc.rows] = nc.k_scale
    vc.reshape(-1, d)[nc.rows] = nc.v_i8
    vs.reshape(-1)[nc.rows] = nc.v_scale
    return kc, ks, vc, vs


def needle_reference(nc: NeedleCase, limit: int, start: int = 0) -> np.ndarray:
    """Closed-form float64 attention ``[Hq, D]`` of ``nc.q`` over positions
    ``[start, limit)``: each background token weighs ``e^0`` with V ``u``,
    each visible needle ``e^s`` with its own V."""
    h = O.hadamard_matrix(nc.head_dim)
    k = (nc.k_i8.astype(np.float64) * nc.k_scale.astype(np.float64)[:, None]) @ h
    v = nc.v_i8.astype(np.float64) * nc.v_scale.astype(np.float64)[:, None]
    s = nc.scale * nc.q.astype(np.float64) @ k.T
    seen = (nc.pos >= start) & (nc.pos < limit)
    s = np.where(seen[None, :], s, -np.inf)
    n_bg = (limit - start) - int(seen.sum())
    mx = np.maximum(s.max(axis=1, keepdims=True), 0.0)
    w = np.exp(s - mx)
    wb = n_bg * np.exp(-mx)
    u = nc.u_i8.astype(np.float64) / 128
    return (w @ v + wb * u[None, :]) / (w.sum(axis=1, keepdims=True) + wb)
