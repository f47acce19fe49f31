"""GPU parity at the size limits the C ABI accepts, through the C ABI.

* Batches past the 1024 rows whose context lengths the decode keeps in LDS,
  up to the 65535-row maximum: rows of length 0 and 1 checked in closed form
  over the whole batch (no key: zeros; one key: softmax weight 1, so its V),
  the others against the oracle on a sample of rows.
* One sequence of 2^18 tokens beside short rows, split across every
  workgroup and recombined: decode, the fused decode-append and a chunk
  verify against the oracle.
* Pools just under the 4 GiB one buffer descriptor addresses, and 6 GiB pools
  (addressed through descriptors rebased per tile, and 64-bit pointers for
  appends): rows whose blocks sit at the top of the pool, on both sides of
  byte offset 2^31 or 2^32 and at the bottom, against the oracle on a compact
  copy of those blocks; and one sequence through every block of such a pool
  (33,554,176 or 50,331,648 tokens) whose output has a closed form.

The caches are filled by the GPU append (bit-exact against the oracle in
test_gpu_kernels.py and again here) and read back for the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import empty_int8_cache, empty_k8v3_cache, make_case, make_needle_case, needle_reference
from tests.kvgpu import (CODEBOOK, DEV, KINDS, alloc, append, assert_close, decode, decode_append, decode_plan, layer, t,
                         to_np, verify)

pytestmark = pytest.mark.gpu


def _oracle_fill(kind, case, keep=None):
    """Oracle cache (numpy) holding the case's tokens (those under `keep`)."""
    sel = slice(None) if keep is None else keep
    if kind == "int8":
        c = empty_int8_cache(case)
        O.quantize_kv_write_paged(case.k[sel], case.v[sel], *c, case.slots[sel])
    else:
        c = empty_k8v3_cache(case)
        O.k8v3_write_paged(case.k[sel], case.v[sel], *c, CODEBOOK, case.slots[sel])
    return c


def _last_tokens(case):
    """Mask of every token but each row's last (in the case's token order) and
    the last tokens' K and V ``[B, Hkv, D]`` (zeros for empty rows)."""
    has = case.lens > 0
    last = np.cumsum(case.lens) - 1
    keep = np.ones(len(case.slots), bool)
    keep[last[has]] = False
    k_new = np.zeros((case.batch, case.num_kv_heads, case.head_dim), np.float16)
    v_new = np.zeros_like(k_new)
    k_new[has] = case.k[last[has]]
    v_new[has] = case.v[last[has]]
    return keep, k_new, v_new


def _v_rows(kind, cache, blk, off):
    """float64 V ``[n, Hkv, D]`` stored at position ``off[i]`` of block ``blk[i]``."""
    if kind == "int8":
        return cache[2][blk, :, off].astype(np.float64) * cache[3][blk, :, off][..., None]
    d = cache[0].shape[-1]
    codes = O.unpack_indices_lowbit(cache[2][blk, :, off], 3, d).astype(np.int64)
    return np.asarray(CODEBOOK, np.float64)[codes] * cache[3][blk, :, off][..., :1].astype(np.float64)


def _assert_same_bytes(got, ref, what):
    for a, b, name in zip(got, ref, ("k_cache", "k_scale", "v", "v_scale")):
        assert np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8)), \
            f"{what}: {name} differs from the oracle's append"


# ---------------------------------------------------------------------------
# batch
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("kind,batch", [("int8", 1025), ("int8", 65535), ("k8v3", 65535)])
def test_decode_batch_limits(kind, batch):
    """Rows from 1024 on read their context length from global memory; 65535
    rows is the largest batch the decode accepts."""
    hq, hkv, d, bs = 8, 2, 128, 16
    rng = np.random.default_rng(700 + batch)
    lens = rng.integers(0, 7 if kind == "int8" else 4, size=batch)
    lens[:3] = [0, 1, 5]
    lens[-3:] = [5, 1, 0]
    case = make_case(710 + batch, batch, hq, hkv, d, bs, lens)
    keep, k_new, v_new = _last_tokens(case)
    cache = alloc(kind, case.num_blocks, hkv, bs, d)
    append(kind, t(case.k[keep]), t(case.v[keep]), cache, t(case.slots[keep]))
    q, bt, cl = t(case.q), t(case.block_table), t(lens.astype(np.int32))
    max_ctx = int(lens.max())
    fused = to_np(decode_append(kind, q, t(k_new), t(v_new), cache, bt, cl, bs, max_ctx, case.scale).float())
    full = tuple(to_np(x) for x in cache)
    _assert_same_bytes(full, _oracle_fill(kind, case), f"{kind} batch {batch}")
    out = to_np(decode(kind, q, cache, bt, cl, bs, max_ctx, case.scale).float())
    assert np.array_equal(fused, out), "fused decode-append differs from append + decode"

    assert not out[lens == 0].any(), "rows with no key must be zeros"
    one = np.nonzero(lens == 1)[0]
    v1 = _v_rows(kind, full, case.block_table[one, 0], np.zeros(len(one), np.int64))
    assert_close(out[one], np.repeat(v1, hq // hkv, axis=1), f"{kind} batch {batch}: one-key rows")

    pick = np.concatenate([np.arange(8), np.arange(1016, 1032), np.arange(batch - 8, batch),
                           rng.choice(batch, 200, replace=False)])
    idx = np.unique(pick[pick < batch])
    ref = O.paged_decode(case.q[idx], layer(kind, full), case.block_table[idx], lens[idx], case.scale)
    assert_close(out[idx], ref, f"{kind} batch {batch}: sampled rows")


# ---------------------------------------------------------------------------
# one long sequence
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("kind", KINDS)
def test_one_long_sequence(kind):
    """A 2^18-token row beside short ones: its context is split across every
    workgroup and recombined in the launch."""
    hq, hkv, d, bs, nq = 8, 2, 128, 256, 16
    lens = np.array([1 << 18, 1, 3000, 17])
    case = make_case(720, len(lens), hq, hkv, d, bs, lens, outlier_channels=2)
    keep, k_new, v_new = _last_tokens(case)
    cache = alloc(kind, case.num_blocks, hkv, bs, d)
    append(kind, t(case.k[keep]), t(case.v[keep]), cache, t(case.slots[keep]))
    q, bt, cl = t(case.q), t(case.block_table), t(lens.astype(np.int32))
    max_ctx = int(lens.max())
    fused = to_np(decode_append(kind, q, t(k_new), t(v_new), cache, bt, cl, bs, max_ctx, case.scale).float())
    full = tuple(to_np(x) for x in cache)
    if kind == "int8":
        _assert_same_bytes(full, _oracle_fill(kind, case), "long row")
    else:
        # the oracle's Lloyd-Max search is slow on the CPU: every row's last
        # token (written by the fused launch) and a sample of the others
        rng = np.random.default_rng(721)
        sample = np.zeros(len(case.slots), bool)
        sample[rng.choice(len(case.slots), 4096, replace=False)] = True
        sample |= ~keep
        ref = _oracle_fill(kind, case, keep=sample)
        s = case.slots[sample]
        blk, off = s // bs, s % bs
        _assert_same_bytes([x[blk, :, off] for x in full], [x[blk, :, off] for x in ref], "long row (sampled)")
    out = to_np(decode(kind, q, cache, bt, cl, bs, max_ctx, case.scale).float())
    assert np.array_equal(fused, out), "fused decode-append differs from append + decode"
    lc = layer(kind, full)
    assert_close(out, O.paged_decode(case.q, lc, case.block_table, lens, case.scale), f"{kind} long row decode")

    # chunk verify: each row's last (up to) 16 tokens as queries
    prefix = np.maximum(lens - nq, 0)
    qlens = (lens - prefix).astype(np.int32)
    qv = np.random.default_rng(722).standard_normal((len(lens), hq, nq, d)).astype(np.float16)
    got = verify(kind, t(qv), cache, bt, t(prefix.astype(np.int32)), t(qlens), bs, max_ctx, case.scale)
    ref = O.paged_verify(qv, lc, case.block_table, prefix, case.scale, query_lens=qlens)
    assert_close(to_np(got.float()), ref, f"{kind} long row verify")


# ---------------------------------------------------------------------------
# 4 GiB pools
# ---------------------------------------------------------------------------

def _edge_ids(case, nblk, specials, rng):
    """Compact block -> pool block: the longest row's last block (its new
    token) is the pool's last, the next used blocks take `specials`, the rest
    random free blocks."""
    bs = case.block_size
    need = (case.lens + bs - 1) // bs
    ids = np.full(case.num_blocks, -1, np.int64)
    ids[case.block_table[0, need[0] - 1]] = nblk - 1
    used = [int(case.block_table[b, i]) for b in range(case.batch) for i in range(need[b])]
    rest = [c for c in used if ids[c] < 0]
    for c, blk in zip(rest, specials):
        ids[c] = blk
    ids[ids < 0] = rng.choice(np.setdiff1d(np.arange(nblk), ids[ids >= 0]), int((ids < 0).sum()), replace=False)
    return ids


# (pool blocks, pool blocks of interest) at Hkv 2, block 256, D 128 (64 KiB of K per block)
POOLS = {
    "under_4gib": (65535, (32768, 32767, 0, 65533, 1)),            # 4,294,901,760 K bytes; blocks at 2 GiB
    "6gib": (98304, (65536, 65535, 32768, 0, 98302)),              # 6 GiB: blocks on either side of 4 GiB
}


@pytest.mark.parametrize("pool", sorted(POOLS))
@pytest.mark.parametrize("kind", KINDS)
def test_rows_at_the_edges_of_a_large_pool(kind, pool):
    """Rows of a pool just under 4 GiB (one buffer descriptor spans it) and of
    a 6 GiB pool (tiles through descriptors rebased per tile, appends through
    64-bit pointers) whose blocks are the pool's last (holding the longest
    row's new token), the blocks on either side of byte offset 2^31 or 2^32,
    the first, and random others; append, fused decode-append, decode and
    chunk verify against the oracle on a compact copy of those blocks."""
    hq, hkv, d, bs, nq = 8, 2, 128, 256, 8
    nblk, specials = POOLS[pool]
    lens = np.array([2000, 300, 257, 9])
    case = make_case(730, len(lens), hq, hkv, d, bs, lens, outlier_channels=2)
    ids = _edge_ids(case, nblk, specials, np.random.default_rng(731))
    bt = ids[case.block_table].astype(np.int32)
    slots = (ids[case.slots // bs] * bs + case.slots % bs).astype(np.int32)

    cache = alloc(kind, nblk, hkv, bs, d)
    try:
        keep, k_new, v_new = _last_tokens(case)
        append(kind, t(case.k[keep]), t(case.v[keep]), cache, t(slots[keep]))
        q, btt, cl = t(case.q), t(bt), t(lens.astype(np.int32))
        max_ctx = int(lens.max())
        fused = to_np(decode_append(kind, q, t(k_new), t(v_new), cache, btt, cl, bs, max_ctx, case.scale).float())
        # the planned launch (its first tiles through the plan's rows; the
        # append rewrites the same bytes): the same output
        plan = decode_plan(kind, cache, btt, cl, bs, hq, max_ctx)
        planned = to_np(decode_append(kind, q, t(k_new), t(v_new), cache, btt, cl, bs, max_ctx, case.scale,
                                      plan=plan).float())
        assert np.array_equal(planned, fused), f"{kind} {pool}: the planned step differs"
        compact = tuple(to_np(x.index_select(0, t(ids))) for x in cache)
        _assert_same_bytes(compact, _oracle_fill(kind, case), f"{kind} {pool} pool")
        out = to_np(decode(kind, q, cache, btt, cl, bs, max_ctx, case.scale).float())
        assert np.array_equal(fused, out), "fused decode-append differs from append + decode"
        lc = layer(kind, compact)
        assert_close(out, O.paged_decode(case.q, lc, case.block_table, lens, case.scale), f"{kind} {pool} decode")
        prefix = lens - nq
        qv = np.random.default_rng(732).standard_normal((len(lens), hq, nq, d)).astype(np.float16)
        got = verify(kind, t(qv), cache, btt, t(prefix.astype(np.int32)), None, bs, max_ctx, case.scale)
        ref = O.paged_verify(qv, lc, case.block_table, prefix, case.scale)
        assert_close(to_np(got.float()), ref, f"{kind} {pool} verify")
        if pool == "6gib":  # SnapKV scores of the longest row, whose blocks include the pool's last
            need = (int(lens[0]) + bs - 1) // bs
            qs = torch.randn(hq, d, generator=torch.Generator(device=DEV).manual_seed(733), device=DEV)
            got = to_np(ops.snapkv_scores_paged(qs, cache[0], cache[1], bt[0, :need].tolist(), int(lens[0]), hq))
            want = O.snapkv_scores_paged(to_np(qs), O.LayerCache(compact[0], compact[1]),
                                         case.block_table[0, :need], int(lens[0]), hq)
            assert np.max(np.abs(got - want) / np.maximum(want, 1e-30)) < 2e-4
    finally:
        del cache
        torch.cuda.empty_cache()


def test_large_pool_needs_blocks_of_32():
    """Past 4 GiB per tensor the decode and verify rebase a descriptor per
    tile, which needs tiles inside one block: block_size 16 is refused."""
    hkv, d, bs = 2, 128, 16
    nblk = (1 << 32) // (hkv * bs * d) + 1
    cache = alloc("int8", nblk, hkv, bs, d)
    try:
        q = torch.zeros((1, 8, 1, d), dtype=torch.float16, device=DEV)
        bt = torch.zeros((1, 1), dtype=torch.int32, device=DEV)
        cl = torch.ones(1, dtype=torch.int32, device=DEV)
        with pytest.raises(RuntimeError, match="block_size >= 32"):
            ops.attn_paged_decode_cached(q, *cache, bt, cl, bs, max_context_len=1, scale=0.1)
        with pytest.raises(RuntimeError, match="block_size >= 32"):
            ops.attn_paged_verify(q, *cache, bt, torch.zeros(1, dtype=torch.int32, device=DEV), bs,
                                  max_context_len=1, scale=0.1)
    finally:
        del cache
        torch.cuda.empty_cache()


WHOLE_POOLS = {"under_4gib": ((1 << 32) - 1) // (256 * 128), "6gib": 3 * (1 << 31) // (256 * 128)}


def _whole_pool(nblk):
    """One sequence over every block of an int8 pool of `nblk` blocks at Hkv 1,
    block 256, D 128 (131071 blocks: the largest under 4 GiB; 196608: 6 GiB),
    in a shuffled block order whose last position is the pool's final row.
    Background keys are zero (score 0) with one constant V row; eight needle
    keys, one per q head, sit at the pool's first and last rows, on either side
    of byte offset 2^31 and of 2^32 (or near the end of a smaller pool), at the
    sequence's first position and elsewhere.  Head h scores its
    needle near ln(n) and the others near 0, so needle and background carry
    comparable weight and the output has a closed form (pinned against the
    oracle on a small pool in test_limit_cases.py).
    Returns the case and its cache tensors (k, k_scale, v, v_scale)."""
    hq, d, bs = 8, 128, 256
    half = (1 << 31) // (bs * d)  # the first block at or past 2 GiB
    top = min(2 * half, nblk - 1)  # the first block at or past 4 GiB, when the pool reaches it
    nc = make_needle_case(740, nblk, bs, d, hq, [(0, 0), (half, 0), (half - 1, bs - 1), (top, 128),
                                                 (top - 1, 17)])
    assert nc.rows[0] == nblk * bs - 1
    kc = torch.zeros((nblk, 1, bs, d), dtype=torch.int8, device=DEV)
    ks = torch.full((nblk, 1, bs), 1 / 128, dtype=torch.float32, device=DEV)
    vc = t(nc.u_i8).view(1, 1, 1, d).expand(nblk, 1, bs, d).contiguous()
    vs = torch.full((nblk, 1, bs), 1 / 128, dtype=torch.float32, device=DEV)
    r = t(nc.rows)
    kc.view(-1, d)[r] = t(nc.k_i8)
    ks.view(-1)[r] = t(nc.k_scale)
    vc.view(-1, d)[r] = t(nc.v_i8)
    vs.view(-1)[r] = t(nc.v_scale)
    return nc, [kc, ks, vc, vs]


@pytest.mark.parametrize("pool", sorted(WHOLE_POOLS))
def test_decode_through_a_whole_pool(pool):
    """Decode over the whole-pool sequence, then the fused decode-append
    rewriting its last position (the pool's final row)."""
    nc, cache = _whole_pool(WHOLE_POOLS[pool])
    try:
        kc, ks, vc, vs = cache
        n, d, bs = nc.n, nc.head_dim, nc.block_size
        q, btt, cl = t(nc.q[None]), t(nc.block_table[None]), t(np.array([n], np.int32))
        out = ops.attn_paged_decode_cached(q, kc, ks, vc, vs, btt, cl, bs, max_context_len=n, scale=nc.scale)
        assert_close(to_np(out.float())[0], needle_reference(nc, n), "whole-pool decode")

        rng = np.random.default_rng(741)
        k_new = rng.standard_normal((1, 1, d)).astype(np.float16)
        v_new = rng.standard_normal((1, 1, d)).astype(np.float16)
        out = ops.attn_paged_decode_append(q, t(k_new), t(v_new), kc, ks, vc, vs, btt, cl, bs, max_context_len=n,
                                           scale=nc.scale)
        one = (np.zeros((1, 1, bs, d), np.int8), np.ones((1, 1, bs), np.float32),
               np.zeros((1, 1, bs, d), np.int8), np.ones((1, 1, bs), np.float32))
        O.quantize_kv_write_paged(k_new, v_new, *one, np.array([bs - 1], np.int32))
        want = tuple(x[0, 0, -1:] for x in one)
        last = t(nc.rows[:1])
        got = (to_np(kc.view(-1, d)[last]), to_np(ks.view(-1)[last]), to_np(vc.view(-1, d)[last]),
               to_np(vs.view(-1)[last]))
        _assert_same_bytes(got, want, "whole-pool fused append")
        nc.k_i8[0], nc.k_scale[0], nc.v_i8[0], nc.v_scale[0] = want[0][0], want[1][0], want[2][0], want[3][0]
        assert_close(to_np(out.float())[0], needle_reference(nc, n), "whole-pool fused decode-append")
        # planned (the append rewrites the same bytes): the same output
        plan = ops.attn_paged_decode_plan(kc, btt, cl, bs, num_q_heads=q.shape[1], max_context_len=n)
        again = ops.attn_paged_decode_append(q, t(k_new), t(v_new), kc, ks, vc, vs, btt, cl, bs, max_context_len=n,
                                             scale=nc.scale, plan=plan)
        assert torch.equal(again, out), "whole-pool planned decode-append differs"
    finally:
        cache.clear()
        torch.cuda.empty_cache()


@pytest.mark.parametrize("pool", sorted(WHOLE_POOLS))
def test_window_verify_through_a_whole_pool(pool):
    """The same chain verify with a window of a third of the sequence: query
    s sees positions [n - 4 - window, n - 4 + s], with needles on both sides
    of the window start (the 32-row kernel under 4 GiB, the 16-row kernel
    with descriptors rebased per tile at 6 GiB)."""
    nc, cache = _whole_pool(WHOLE_POOLS[pool])
    try:
        kc, ks, vc, vs = cache
        n, d, bs, hq, nq = nc.n, nc.head_dim, nc.block_size, len(nc.pos), 4
        window = n // 3
        lo = n - nq - window
        assert (nc.pos < lo).any() and (nc.pos >= lo).any(), "needles on both sides of the window start"
        qv = np.ascontiguousarray(np.broadcast_to(nc.q[:, None, :], (hq, nq, d)))
        got = to_np(ops.attn_paged_verify(t(qv[None]), kc, ks, vc, vs, t(nc.block_table[None]),
                                          t(np.array([n - nq], np.int32)), bs, max_context_len=n,
                                          scale=nc.scale, window=window).float())[0]
        for s in range(nq):
            assert_close(got[:, s], needle_reference(nc, n - nq + s + 1, start=lo), f"whole-pool window verify {s}")
    finally:
        cache.clear()
        torch.cuda.empty_cache()


@pytest.mark.parametrize("pool", sorted(WHOLE_POOLS))
def test_chain_verify_through_a_whole_pool(pool):
    """A 4-query chain verify of the whole-pool sequence's last positions:
    query s sees positions [0, n - 4 + s].  The single query block's 33.5M
    keys are split across workgroups (no workgroup accumulates more than 2^20
    in fp32, whose rounding would otherwise drift past the tolerance)."""
    nc, cache = _whole_pool(WHOLE_POOLS[pool])
    try:
        kc, ks, vc, vs = cache
        n, d, bs, hq, nq = nc.n, nc.head_dim, nc.block_size, len(nc.pos), 4
        qv = np.ascontiguousarray(np.broadcast_to(nc.q[:, None, :], (hq, nq, d)))
        got = to_np(ops.attn_paged_verify(t(qv[None]), kc, ks, vc, vs, t(nc.block_table[None]),
                                          t(np.array([n - nq], np.int32)), bs, max_context_len=n,
                                          scale=nc.scale).float())[0]
        for s in range(nq):
            assert_close(got[:, s], needle_reference(nc, n - nq + s + 1), f"whole-pool verify query {s}")
    finally:
        cache.clear()
        torch.cuda.empty_cache()
