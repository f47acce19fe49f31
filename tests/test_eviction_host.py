"""Eviction policy arithmetic against the reference's own ``KVEviction``
(outputs recorded by tests/golden/make_bookkeeping_traces.py): block bytes,
Ada-KV budgets, the DuoAttention split, the recall gate, the config
defaults, and the disabled-eviction no-op.  Host only."""

from __future__ import annotations

import dataclasses
import json
from pathlib import Path

import pytest
import torch

from superl8_serve_amd.eviction import EvictionConfig, KVEviction
from superl8_serve_amd.paged_cache import PagedKVCache

FIX = json.loads((Path(__file__).resolve().parent / "golden" / "bookkeeping_traces.json").read_text())


def test_block_bytes_match_the_reference():
    for h, b, d, vq, want in FIX["block_bytes"]:
        assert KVEviction.block_bytes(h, b, d, v_quant=vq) == want
    # the reference tests' own pins (tests/test_kv_eviction.py:66-77)
    assert KVEviction.block_bytes(8, 16, 128) == 2 * 8 * 16 * 128 + 2 * 8 * 16 * 4
    assert KVEviction.block_bytes(2, 8, 32) == 1024 + 128


def test_adakv_budgets_match_the_reference():
    for n, t, lo, hi, want in FIX["adakv"]:
        assert KVEviction.adakv_budgets(n, t, lo, hi) == want


def test_duoattn_split_matches_the_reference():
    for h, f, streaming, rest in FIX["duoattn"]:
        assert KVEviction.duoattn_split(h, f) == (streaming, rest)


def test_recall_gate_matches_the_reference():
    for case in FIX["recall"]:
        got = KVEviction.recall_check(torch.tensor(case["a"]), torch.tensor(case["b"]), case["threshold"])
        assert got["passed"] == case["passed"] and got["threshold"] == case["threshold"]
        assert got["cos_sim"] == pytest.approx(case["cos_sim"], rel=1e-6, abs=1e-7)


def test_config_defaults_are_the_references():
    want = dict(enabled=False, policy="snapkv", kv_budget=512, recall_threshold=0.99, measure_hbm=True,
                adakv_min_budget=128, adakv_max_budget=1024, duoattn_streaming_heads=0.25, duoattn_window=128)
    assert dataclasses.asdict(EvictionConfig()) == want


def test_disabled_eviction_touches_nothing():
    cache = PagedKVCache(2, 4, 2, 64, 32, device="cpu", block_size=4)
    slot = cache.alloc()
    cache.ensure_capacity([slot], [16])
    before = (list(cache._slot_blocks[slot]), list(cache._free_blocks), dict(cache._block_refcount))
    res = cache.evict_after_prefill(slot, 16, eviction_config=EvictionConfig(enabled=False), num_heads=4)
    assert res == {"evicted": False, "strategy": None, "metrics": None, "recall": None}
    assert (list(cache._slot_blocks[slot]), list(cache._free_blocks), dict(cache._block_refcount)) == before


def test_compact_no_ops_need_no_kernel():
    """Empty keep lists and keep lists that would not free a block return
    the reference's no-op metrics without moving anything."""
    cache = PagedKVCache(2, 4, 2, 64, 32, device="cpu", block_size=4)
    slot = cache.alloc()
    cache.ensure_capacity([slot], [8])
    assert KVEviction.compact(cache, slot, []) == {"bytes_freed": 0, "blocks_freed": 0, "blocks_after": 2,
                                                    "tokens_kept": 0}
    assert KVEviction.compact(cache, slot, list(range(8))) == {"bytes_freed": 0, "blocks_freed": 0,
                                                                "blocks_after": 2, "tokens_kept": 8}
    empty = cache.alloc()
    assert KVEviction.compact(cache, empty, [0, 1]) == {"bytes_freed": 0, "blocks_freed": 0, "blocks_after": 0,
                                                         "tokens_kept": 0}


def test_oracle_snapkv_selection_matches_the_reference():
    """The oracle's SnapKV ranking picks exactly the reference's positions on
    the recorded inputs (which pins it for the GPU scoring tests)."""
    import numpy as np

    from oracle import kv_oracle as O

    for case in FIX["snapkv"]:
        q, k = np.asarray(case["q"]), np.asarray(case["k"])
        scores = O.snapkv_scores(q, k, case["num_heads"], case["num_kv_heads"])
        assert O.snapkv_select(scores, case["budget"]) == case["selected"]
        assert abs(scores.sum() - 1.0) < 1e-12  # a mean of softmax rows


def test_oracle_gather_slots_moves_rows_only():
    import numpy as np

    from oracle import kv_oracle as O

    rng = np.random.default_rng(0)
    t = rng.integers(-128, 128, size=(3, 6, 2, 4, 8)).astype(np.int8)
    u = t.copy()
    src, dst = [1, 5, 22], [16, 17, 18]
    O.gather_slots([u], src, dst)
    for j, (s, d) in enumerate(zip(src, dst)):
        assert np.array_equal(u[:, d // 4, :, d % 4], t[:, s // 4, :, s % 4])
    keep = np.ones((6, 4), bool)
    for d in dst:
        keep[d // 4, d % 4] = False
    assert np.array_equal(u.transpose(1, 3, 0, 2, 4)[keep], t.transpose(1, 3, 0, 2, 4)[keep])


def test_defragment_after_compaction_packs_every_live_block(monkeypatch):
    """Compaction takes its new blocks from the pool without refcount entries
    (as the reference's does); a later ``defragment`` must still move them
    below the used watermark.  The byte moves run on host stand-ins built
    from the oracle's copy and gather, so every token can be followed."""
    import numpy as np

    from oracle import kv_oracle as O
    from superl8_serve_amd import ops

    monkeypatch.setattr(ops, "copy_blocks",
                        lambda ts, src, dst: O.copy_blocks([t.numpy() for t in ts], list(src), list(dst)))
    monkeypatch.setattr(ops, "gather_slots",
                        lambda ts, src, dst, bs: O.gather_slots([t.numpy() for t in ts], list(src), list(dst)))
    bs = 4
    c = PagedKVCache(num_layers=2, num_slots=4, num_kv_heads=2, max_len=32, head_dim=32, device="cpu",
                     block_size=bs)
    rng = np.random.default_rng(5)
    c.k_cache.copy_(torch.from_numpy(rng.integers(-127, 128, size=tuple(c.k_cache.shape), dtype=np.int8)))
    c.v_cache.copy_(torch.from_numpy(rng.integers(-127, 128, size=tuple(c.v_cache.shape), dtype=np.int8)))
    a, b, d = c.alloc(), c.alloc(), c.alloc()
    c.ensure_capacity([a, b, d], [20, 12, 16])
    keep = [0, 3, 5, 9, 10, 17]
    token = lambda s, p: (c.k_cache[:, c._slot_blocks[s][p // bs], :, p % bs].clone(),  # noqa: E731
                          c.v_cache[:, c._slot_blocks[s][p // bs], :, p % bs].clone())
    want_a = [token(a, p) for p in keep]
    want_d = [token(d, p) for p in range(16)]
    KVEviction.compact(c, a, keep)                       # a's new blocks carry no refcount entry
    assert any(blk not in c._block_refcount for blk in c._slot_blocks[a])
    c.free(b)
    moves = c.defragment()
    assert moves
    live = {blk for s in (a, d) for blk in c._slot_blocks[s]}
    assert len(live) == c.used_blocks and max(live) < c.used_blocks
    assert set(c._free_blocks) == set(range(c.used_blocks, c.num_blocks))
    for j, (k0, v0) in enumerate(want_a):
        k1, v1 = token(a, j)
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
    for p, (k0, v0) in enumerate(want_d):
        k1, v1 = token(d, p)
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
