"""GPU tests of prompt-time eviction through the C ABI: SnapKV scoring over a
dense K and over the paged int8 cache against the oracle, the reference's
recorded selections, keep-list compaction (byte moves) against the oracle's
gather and the reference's recorded bookkeeping, and the full
``evict_after_prefill`` flow on the reference's recorded scenarios.

Reference pins reproduced: a full keep leaves the cache bit-identical
(tests/test_kv_eviction.py:464-479); 3 blocks -> 1 frees exactly
2 x 2 x block_bytes (tests/test_kv_eviction.py:424-441)."""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from superl8_serve_amd.eviction import EvictionConfig, KVEviction
from superl8_serve_amd.paged_cache import PagedKVCache

pytestmark = pytest.mark.gpu

DEV = "cuda"
FIX = json.loads((Path(__file__).resolve().parent / "golden" / "bookkeeping_traces.json").read_text())


def _np(t):
    return t.detach().cpu().numpy()


def _same(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def _fill(cache, slot, n, seed, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    for layer in range(cache.num_layers):
        k = (torch.randn(1, cache.num_kv_heads, n, cache.head_dim, generator=g, device=DEV) * scale).half()
        v = (torch.randn(1, cache.num_kv_heads, n, cache.head_dim, generator=g, device=DEV) * scale).half()
        cache.write_prefill(layer, k, v, slot=slot)


@pytest.mark.parametrize("case", range(len(FIX["snapkv"])))
def test_snapkv_selection_reproduces_the_reference(case):
    c = FIX["snapkv"][case]
    q = torch.tensor(c["q"], device=DEV)
    k = torch.tensor(c["k"], device=DEV)
    if c["layout"] == "4d":
        q, k = q.reshape(1, c["num_heads"], 1, -1), k.unsqueeze(0)
    sel = KVEviction.snapkv_selection(q, k, c["budget"], c["num_heads"], c["num_kv_heads"])
    assert sel == c["selected"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("hq,hkv,d,s", [(32, 8, 128, 1000), (4, 4, 64, 33), (16, 2, 256, 500), (8, 1, 32, 7)])
def test_snapkv_scores_dense_against_the_oracle(dtype, hq, hkv, d, s):
    g = torch.Generator(device=DEV).manual_seed(hq * 7 + s)
    q = torch.randn(hq, d, generator=g, device=DEV).to(dtype)
    k = torch.randn(hkv, s, d, generator=g, device=DEV).to(dtype)
    got = _np(ops.snapkv_scores(q, k, hq, hkv))
    want = O.snapkv_scores(_np(q.float()), _np(k.float()), hq, hkv)
    assert np.max(np.abs(got - want) / np.maximum(want, 1e-30)) < 2e-5
    assert abs(got.sum() - 1.0) < 1e-4


@pytest.mark.parametrize("v_quant", ["int8", "lloydmax3"])
@pytest.mark.parametrize("bs,d", [(16, 128), (4, 64), (256, 128), (8, 256)])
def test_snapkv_scores_paged_against_the_oracle(v_quant, bs, d):
    if v_quant == "lloydmax3" and d < 128:
        pytest.skip("the K8V3 layout needs head_dim 128 or 256")
    hq, hkv, n = 16, 4, 700
    cache = PagedKVCache(2, 3, hkv, 1024, d, device=DEV, block_size=bs, v_quant=v_quant)
    other = cache.alloc()
    cache.ensure_capacity([other], [bs + 3])  # interleave another slot's blocks
    slot = cache.alloc()
    cache.ensure_capacity([slot], [n])
    _fill(cache, slot, n, 5, scale=2.0)
    q = torch.randn(hq, d, generator=torch.Generator(device=DEV).manual_seed(6), device=DEV) * 2
    got = _np(ops.snapkv_scores_paged(q, cache.k_cache[1], cache.k_scale[1], cache._slot_blocks[slot], n, hq))
    layer = O.LayerCache(_np(cache.k_cache[1]), _np(cache.k_scale[1]))  # K only: scoring reads no V
    want = O.snapkv_scores_paged(_np(q), layer, cache._slot_blocks[slot], n, hq)
    assert np.max(np.abs(got - want) / np.maximum(want, 1e-30)) < 2e-4
    # the same ranking as scoring the dense read-back of the cache
    kd, _ = cache.read_dense(1, slot, n, dtype=torch.float32)
    dense = _np(ops.snapkv_scores(q, kd, hq, hkv))
    assert np.max(np.abs(got - dense) / np.maximum(dense, 1e-30)) < 2e-3
    budget = 100
    sel = KVEviction.snapkv_selection_paged(cache, 1, slot, n, q, budget, hq)
    ref = O.snapkv_select(want, budget)
    if sel != ref:  # only near-ties at the cut may differ
        cut = np.sort(want)[::-1][budget - 1]
        for p in set(sel) ^ set(ref):
            assert abs(want[p] - cut) <= 1e-4 * cut


@pytest.mark.parametrize("case", range(len(FIX["compact"])))
def test_compact_reproduces_the_reference_bookkeeping_and_moves_bytes(case):
    c = FIX["compact"][case]
    layers, slots, hkv, max_len, d, bs, seq_len, keep, extra = c["args"]
    cache = PagedKVCache(layers, slots, hkv, max_len, d, device=DEV, block_size=bs)
    others = []
    for _ in range(extra):
        s = cache.alloc()
        cache.ensure_capacity([s], [bs + 1])
        others.append(s)
    slot = cache.alloc()
    assert (others, slot) == (c["others"], c["slot"])
    cache.ensure_capacity([slot], [seq_len])
    assert cache._slot_blocks[slot] == c["blocks_before"] and cache._free_blocks == c["free_before"]
    _fill(cache, slot, seq_len, 30 + case)
    before = [_np(t) for t in cache._tensors()]
    metrics = KVEviction.compact(cache, slot, list(keep))
    torch.cuda.synchronize()
    assert metrics == c["metrics"]
    assert cache._slot_blocks[slot] == c["blocks_after"] and cache._free_blocks == c["free_after"]
    assert sorted([int(a), int(b)] for a, b in cache._block_refcount.items()) == c["refcount_after"]
    after = [_np(t) for t in cache._tensors()]
    if metrics["blocks_freed"] == 0:  # nothing written (the reference's pin for a full keep)
        for a, b in zip(after, before):
            assert _same(a, b)
        return
    old = c["blocks_before"]
    src = [old[p // bs] * bs + p % bs for p in keep]
    dst = [cache._slot_blocks[slot][j // bs] * bs + j % bs for j in range(len(keep))]
    # the reference writes every layer's kept tokens at these slots, block by block
    assert sum(c["writes"][:len(c["writes"]) // layers], []) == dst
    want = [b.copy() for b in before]
    O.gather_slots(want, src, dst)
    for a, b in zip(after, want):
        assert _same(a, b), "compaction moved other bytes than the kept rows"


def test_full_keep_is_bit_identical_and_bytes_freed_is_exact():
    cache = PagedKVCache(2, 4, 2, 64, 32, device=DEV, block_size=4)
    slot = cache.alloc()
    cache.ensure_capacity([slot], [8])
    _fill(cache, slot, 8, 1, scale=0.1)
    snap = [t.clone() for t in cache._tensors()]
    m = KVEviction.compact(cache, slot, list(range(8)))
    assert m["blocks_freed"] == 0 and all(torch.equal(a, b) for a, b in zip(cache._tensors(), snap))
    cache2 = PagedKVCache(2, 4, 2, 64, 32, device=DEV, block_size=4)
    slot = cache2.alloc()
    cache2.ensure_capacity([slot], [12])
    _fill(cache2, slot, 12, 2, scale=0.1)
    res = cache2.evict_after_prefill(slot, 12, eviction_config=EvictionConfig(enabled=True, kv_budget=4),
                                     num_heads=4, keep_mask=[0, 1, 2, 3])
    assert res["metrics"]["bytes_freed"] == 2 * 2 * KVEviction.block_bytes(2, 4, 32)


@pytest.mark.parametrize("v_quant", ["int8", "lloydmax3"])
def test_compacted_sequence_reads_back_its_kept_tokens_exactly(v_quant):
    """After compaction, position j of the slot holds kept position keep[j]:
    read_dense and the decode attention over the new layout equal the dense
    read and the oracle over the kept tokens of the old layout."""
    hq, hkv, d, bs, n = 8, 2, 128, 16, 150
    cache = PagedKVCache(3, 4, hkv, 512, d, device=DEV, block_size=bs, v_quant=v_quant)
    slot = cache.alloc()
    cache.ensure_capacity([slot], [n])
    _fill(cache, slot, n, 9)
    rng = np.random.default_rng(9)
    keep = sorted(rng.choice(n, 61, replace=False).tolist())
    dense = [[_np(x) for x in cache.read_dense(layer, slot, n)] for layer in range(3)]
    m = KVEviction.compact(cache, slot, keep)
    assert m["tokens_kept"] == 61 and m["blocks_after"] == 4 and m["blocks_freed"] == 6
    for layer in range(3):
        k2, v2 = (_np(x) for x in cache.read_dense(layer, slot, len(keep)))
        assert _same(k2, dense[layer][0][:, :, keep]) and _same(v2, dense[layer][1][:, :, keep])
    q = torch.randn(1, hq, 1, d, device=DEV).half()
    out = cache.decode_attn(1, q, [slot], [len(keep) - 1], scale=1 / math.sqrt(d))
    if v_quant == "int8":
        layer1 = O.LayerCache(*[_np(t[1]) for t in cache._tensors()])
    else:
        t = [_np(x[1]) for x in cache._tensors()]
        layer1 = O.LayerCache(t[0], t[1], v_packed=t[2], v_norm=t[3], v_codebook=_np(cache.v_codebook[1]))
    ref = O.paged_decode(_np(q)[:, :, 0], layer1, np.asarray([cache._slot_blocks[slot]]), np.asarray([len(keep)]),
                         1 / math.sqrt(d))
    mx, rel = O.attention_errors(_np(out.float())[:, :, 0], ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL


@pytest.mark.parametrize("case", range(len(FIX["evict"])))
def test_evict_after_prefill_reproduces_the_reference(case):
    c = FIX["evict"][case]
    cache = PagedKVCache(c["layers"], 4, 2, 64, 32, device=DEV, block_size=c["block_size"])
    slot = cache.alloc()
    cache.ensure_capacity([slot], [c["seq_len"]])
    assert cache._slot_blocks[slot] == c["blocks_before"]
    _fill(cache, slot, c["seq_len"], 100 + case, scale=0.1)
    kw = {}
    if "keep_mask" in c:
        kw["keep_mask"] = c["keep_mask"]
    if "q_last" in c:
        kw["q_last"] = torch.tensor(c["q_last"], device=DEV)
        kw["k_full"] = torch.tensor(c["k_full"], device=DEV)
    if "logits_full" in c:
        kw["logits_full"] = torch.tensor(c["logits_full"])
        kw["logits_fn"] = lambda: torch.tensor(c["logits_after"])
    res = cache.evict_after_prefill(slot, c["seq_len"], eviction_config=EvictionConfig(**c["config"]),
                                    num_heads=c["num_heads"], **kw)
    want = c["result"]
    assert {k: res[k] for k in ("evicted", "strategy", "metrics")} == {k: want[k] for k in
                                                                       ("evicted", "strategy", "metrics")}
    if want["recall"] is None:
        assert res["recall"] is None
    else:
        assert res["recall"]["passed"] == want["recall"]["passed"]
        assert res["recall"]["cos_sim"] == pytest.approx(want["recall"]["cos_sim"], abs=1e-6)
    assert cache._slot_blocks[slot] == c["blocks_after"] and cache._free_blocks == c["free_after"]
