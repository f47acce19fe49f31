"""Host bookkeeping against the reference's own ``PagedKVCache``: the call
sequences recorded from it in tests/golden/bookkeeping_traces.json (by
tests/golden/make_bookkeeping_traces.py, which runs the reference module) are
replayed on ``superl8_serve_amd.paged_cache.PagedKVCache``, and every call's
result and the bookkeeping after it must be identical: free lists (LIFO
order), slot block lists, refcounts, prefix pins, trie entries in the order
the eviction walk visits them (which decides LRU ties), the LRU clock, and
the byte accounting.  Host-only: no kernel runs."""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from superl8_serve_amd.paged_cache import PagedKVCache

FIXTURE = json.loads((Path(__file__).resolve().parent / "golden" / "bookkeeping_traces.json").read_text())


def _entries(cache) -> list:
    """[token path, num_tokens, blocks, lru] in pre-order over children in
    insertion order."""
    out = []
    stack = [([], iter(cache._trie.children.items()))]
    while stack:
        path, it = stack[-1]
        nxt = next(it, None)
        if nxt is None:
            stack.pop()
            continue
        tok, node = nxt
        if node.entry is not None:
            out.append([path + [tok], node.entry.num_tokens, list(node.entry.blocks), node.entry.lru])
        stack.append((path + [tok], iter(node.children.items())))
    return out


def _state(cache) -> dict:
    return {
        "free_blocks": list(cache._free_blocks),
        "free_slots": list(cache._free_slots),
        "slot_blocks": [list(b) for b in cache._slot_blocks],
        "refcount": sorted([int(k), int(v)] for k, v in cache._block_refcount.items()),
        "prefix_refs": sorted([int(k), int(v)] for k, v in cache._prefix_block_refs.items()),
        "entries": _entries(cache),
        "entry_count": cache._prefix_entry_count,
        "lru": cache._lru_clock,
        "used_blocks": cache.used_blocks,
        "pinned_prefix_blocks": cache.pinned_prefix_blocks,
        "prefix_block_bytes": cache.prefix_block_bytes(),
    }


def test_fixture_covers_evictions_and_lru_ties():
    removed = ties = errors = 0
    for tr in FIXTURE["traces"]:
        states = [s["state"] for s in tr["steps"]]
        errors += sum("error" in s for s in tr["steps"])
        for a, b in zip(states, states[1:]):
            gone = {tuple(e[0]) for e in a["entries"]} - {tuple(e[0]) for e in b["entries"]}
            if gone:
                removed += len(gone)
                lrus = [e[3] for e in a["entries"]]
                ties += lrus.count(min(lrus)) > 1
    assert removed >= 20 and ties >= 5 and errors >= 5


@pytest.mark.parametrize("trace", FIXTURE["traces"], ids=lambda t: f"seed{t['seed']}")
def test_trace_replays_identically(trace):
    kw = dict(trace["config"])
    cache = PagedKVCache(1, kw.pop("num_slots"), 2, kw.pop("max_len"), 32, device="cpu", **kw)
    for i, step in enumerate(trace["steps"]):
        op = step["op"]
        where = f"step {i} ({op})"
        try:
            if op == "alloc":
                assert cache.alloc() == step["result"], where
            elif op == "ensure_capacity":
                cache.ensure_capacity(step["slots"], step["lengths"])
            elif op == "store_prefix":
                cache.store_prefix(step["tokens"], step["slot"])
            elif op == "lookup_prefix":
                n, blocks = cache.lookup_prefix(step["tokens"])
                assert [n, list(blocks)] == step["result"], where
                if step.get("then_share") and n > 0:
                    s = cache.alloc()
                    assert s == step["shared_slot"], where
                    cache.share_blocks(s, blocks)
            elif op == "free":
                cache.free(step["slot"])
            elif op == "extend":
                cache.ensure_capacity([step["slot"]], [len(step["tokens"])])
            else:
                raise AssertionError(f"unknown op {op}")
            assert "error" not in step, f"{where}: the reference raised {step.get('error')!r}"
        except RuntimeError as e:
            assert step.get("error") == str(e), f"{where}: raised {e!r}, the reference {step.get('error')!r}"
        got = _state(cache)
        for key, want in step["state"].items():
            assert got[key] == want, f"{where}: {key} differs from the reference\n ours {got[key]}\n ref  {want}"
