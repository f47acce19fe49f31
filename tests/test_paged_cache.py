"""Host bookkeeping of the paged cache (CPU): slots, LIFO block pool,
reference counts, the prefix trie with LRU eviction and its block budget,
slot mappings and block tables -- the behaviour of the reference's
PagedKVCache (superl8serve/engine/kv_cache.py:703-995) read from its source."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import codebook
from superl8_serve_amd.paged_cache import PagedKVCache, _unpack3, block_bytes


def _cache(**kw):
    args = dict(num_layers=2, num_slots=4, num_kv_heads=2, max_len=64, head_dim=32, device="cpu", block_size=4)
    args.update(kw)
    return PagedKVCache(**args)


def test_layout_and_defaults():
    c = _cache()
    assert c.max_blocks_per_seq == 16 and c.num_blocks == 64          # slots x ceil(max_len / bs)
    assert tuple(c.k_cache.shape) == (2, 64, 2, 4, 32) and c.k_cache.dtype == torch.int8
    assert tuple(c.v_scale.shape) == (2, 64, 2, 4) and c.v_scale.dtype == torch.float32
    assert torch.all(c.k_scale == 1) and c._max_prefix_blocks == 32   # half the pool
    h = _cache(v_quant="lloydmax3", head_dim=128)
    assert tuple(h.v_packed.shape) == (2, 64, 2, 4, 12) and tuple(h.v_norm.shape) == (2, 64, 2, 4, 1)
    assert h.v_cache is None and tuple(h.v_codebook.shape) == (2, 8)
    hy = _cache(kv_layers=[3, 7, 11])
    assert hy.num_layers == 3 and hy._layer_row(7) == 1
    with pytest.raises(ValueError):
        _cache(v_quant="fp8")


def test_codebook_matches_oracle():
    assert np.array_equal(codebook.gaussian_codebook(3, 128), O.gaussian_codebook(3, 128))


def test_block_bytes_matches_oracle():
    for v_quant in ("int8", "lloydmax3"):
        for hkv, bs, d in ((8, 16, 128), (4, 16, 256), (8, 256, 128)):
            assert block_bytes(hkv, bs, d, v_quant) == O.block_bytes(hkv, bs, d, v_quant)


def test_lifo_slots_and_blocks():
    c = _cache()
    s0, s1 = c.alloc(), c.alloc()
    assert (s0, s1) == (3, 2)                                  # list.pop() from the end
    c.ensure_capacity([s0, s1], [5, 4])                         # 2 blocks, then 1 block
    assert c._slot_blocks[s0] == [63, 62] and c._slot_blocks[s1] == [61]
    assert c.used_blocks == 3 and c.has_free_block()
    c.free(s0)
    assert c._free_blocks[-2:] == [63, 62] and c._free_slots[-1] == s0
    s2 = c.alloc()
    assert s2 == s0
    c.ensure_capacity([s2], [9])
    assert c._slot_blocks[s2] == [62, 63, 60]                   # last returned is first reused
    c.ensure_capacity([s2], [9])                                # already large enough: no change
    assert c._slot_blocks[s2] == [62, 63, 60]


def test_pool_exhaustion_raises():
    c = _cache(num_blocks=3)
    s = c.alloc()
    with pytest.raises(RuntimeError):
        c.ensure_capacity([s], [13])
    c2 = _cache(num_slots=1)
    c2.alloc()
    assert not c2.has_free_slot()
    with pytest.raises(RuntimeError):
        c2.alloc()


def test_shared_blocks_refcount():
    c = _cache()
    a, b = c.alloc(), c.alloc()
    c.ensure_capacity([a], [8])
    shared = list(c._slot_blocks[a])
    c.share_blocks(b, shared)
    assert all(c._block_refcount[x] == 2 for x in shared)
    c.free(a)
    assert c.used_blocks == 2 and all(c._block_refcount[x] == 1 for x in shared)
    c.free(b)
    assert c.used_blocks == 0 and not c._block_refcount


def test_prefix_store_lookup_and_lru():
    c = _cache()
    s = c.alloc()
    toks = list(range(100, 111))                                # 11 tokens: 2 full blocks
    c.ensure_capacity([s], [len(toks)])
    blocks = list(c._slot_blocks[s])
    c.store_prefix(toks, s)
    assert c._prefix_entry_count == 2 and c.pinned_prefix_blocks == 2
    assert c._block_refcount[blocks[0]] == 3 and c._block_refcount[blocks[1]] == 2  # slot + one per entry
    n, got = c.lookup_prefix(toks[:9] + [999])
    assert n == 8 and got == blocks[:2]
    n, got = c.lookup_prefix(toks[:7])
    assert n == 4 and got == blocks[:1]
    assert c.lookup_prefix([5, 6, 7, 8]) == (0, [])
    assert c.prefix_block_bytes() == 2 * 2 * block_bytes(2, 4, 32)
    # storing again only bumps LRU stamps
    c.store_prefix(toks, s)
    assert c._prefix_entry_count == 2


def test_prefix_entry_cap_evicts_least_recent():
    c = _cache(max_prefix_entries=2)
    a = c.alloc()
    ta = [1, 2, 3, 4, 5, 6, 7, 8]
    c.ensure_capacity([a], [8])
    c.store_prefix(ta, a)                                       # entries at 4 and 8 (stamp 1)
    b = c.alloc()
    tb = [9, 9, 9, 9]
    c.ensure_capacity([b], [4])
    c.lookup_prefix(ta[:4])                                     # stamp 2 on the 4-token entry of ta
    c.store_prefix(tb, b)                                       # cap reached: evict the oldest (ta's 8-token, stamp 1)
    assert c._prefix_entry_count == 2
    assert c.lookup_prefix(ta) == (4, c._slot_blocks[a][:1])
    assert c.lookup_prefix(tb)[0] == 4


def test_prefix_block_budget():
    c = _cache(max_prefix_blocks=3)
    held = []
    for i in range(3):
        s = c.alloc()
        toks = [10 * i + j for j in range(8)]
        c.ensure_capacity([s], [8])
        c.store_prefix(toks, s)
        held.append((s, toks))
        assert c.pinned_prefix_blocks <= 3
    # the oldest sequence's entries were evicted first
    assert c.lookup_prefix(held[0][1])[0] == 0
    assert c.lookup_prefix(held[2][1])[0] == 8
    # eviction only drops the trie's references: live slots keep their blocks
    for s, _ in held:
        assert all(c._block_refcount.get(x, 0) >= 1 for x in c._slot_blocks[s])
    # once the slots finish, evicted-entry blocks return to the pool
    for s, _ in held:
        c.free(s)
    assert c.used_blocks == c.pinned_prefix_blocks


def test_eviction_prunes_empty_trie_nodes():
    c = _cache(max_prefix_entries=1)
    a = c.alloc()
    c.ensure_capacity([a], [4])
    c.store_prefix([1, 2, 3, 4], a)
    b = c.alloc()
    c.ensure_capacity([b], [4])
    c.store_prefix([7, 7, 7, 7], b)                             # evicts [1,2,3,4]'s entry
    node = c._trie.children[1].children[2].children[3]
    assert 4 not in node.children                                # the emptied leaf is removed


def test_slot_mapping_and_block_table():
    c = _cache()
    s = c.alloc()
    c.ensure_capacity([s], [10])
    owned = c._slot_blocks[s]
    assert c.flat_slot_mapping(s, 6) == [owned[p // 4] * 4 + p % 4 for p in range(6)]
    assert c.slot_mapping_for([s, s], [0, 9]).tolist() == [owned[0] * 4, owned[2] * 4 + 1]
    bt = c.block_table([s, c.alloc()])
    assert bt.shape == (2, 16) and bt[0, :3].tolist() == owned and int(bt[0, 3:].abs().sum()) == 0
    assert int(bt[1].abs().sum()) == 0
    dst = torch.zeros(2, 16, dtype=torch.int32)
    c.fill_block_table(dst, [s, s])
    assert dst[1, :3].tolist() == owned
    sm = torch.zeros(2, dtype=torch.int32)
    c.fill_slot_mapping(sm, [s, s], [1, 5])
    assert sm.tolist() == [owned[0] * 4 + 1, owned[1] * 4 + 1]


def test_unpack3_matches_oracle():
    codes = np.random.default_rng(0).integers(0, 8, size=(5, 256)).astype(np.uint8)
    words = O.pack_indices_lowbit(codes, 3)
    got = _unpack3(torch.from_numpy(words), 256).numpy()
    assert np.array_equal(got, codes)
