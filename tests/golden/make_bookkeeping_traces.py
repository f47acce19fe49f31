"""Writes bookkeeping_traces.json: what the reference's own ``PagedKVCache``
and ``KVEviction`` do, recorded by running them.

    python tests/golden/make_bookkeeping_traces.py [reference root]

Run only in the container that holds the reference checkout (default
/root/reference).  ``superl8serve/engine/kv_cache.py`` is loaded by file path;
its ``superl8`` import is satisfied by a CPU stand-in built from this
repository's oracle (``oracle/kv_oracle.py``: the rotation, the int8 append
and the codebook), which is enough for host bookkeeping, whose results never
depend on the numerics.  Nothing else of the reference is imported.

Contents
  traces        seeded sequences of alloc / free / ensure_capacity /
                share_blocks / store_prefix / lookup_prefix calls on small
                pools (entry caps, block budgets, LRU ties), with every call's
                result and the cache's bookkeeping after it: free lists, slot
                blocks, refcounts, prefix pins, trie entries in the order the
                reference's eviction walk visits them, LRU clock.
  block_bytes   KVEviction.block_bytes over a grid of geometries.
  adakv         KVEviction.adakv_budgets over a grid of arguments.
  duoattn       KVEviction.duoattn_split over a grid of arguments.
  snapkv        KVEviction.snapkv_selection on seeded q / K (inputs stored).
  recall        KVEviction.recall_check on small logit vectors.
  compact       KVEviction.compact scenarios: metrics, the blocks the slot
                ends with, free list and refcounts after, and the
                (kept position -> new flat slot) mapping of its rewrite.
  evict         PagedKVCache.evict_after_prefill scenarios (policies, keep
                masks, recall gate): the returned dict and the slot's blocks.
  shim_import   the module also imports with this repository's ``superl8``
                interface installed, and the names it binds at import.
"""

from __future__ import annotations

import importlib.util
import json
import sys
import types
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import kv_oracle as O  # noqa: E402

OUT = Path(__file__).resolve().parent / "bookkeeping_traces.json"
STUB_NAMES = ("superl8", "superl8.quant", "superl8.quant.rotation", "superl8.quant.lloydmax")


def _install_cpu_stub(calls: list) -> None:
    st = types.ModuleType("superl8")
    qm = types.ModuleType("superl8.quant")
    rm = types.ModuleType("superl8.quant.rotation")
    lm = types.ModuleType("superl8.quant.lloydmax")

    def rotate_last(x):
        return torch.from_numpy(O.rotate_last(x.detach().cpu().numpy()))

    def quantize_kv_write_paged(k, v, k_cache, k_scale, v_cache, v_scale, slot_mapping):
        sm = slot_mapping.detach().cpu().numpy().astype(np.int64)
        calls.append(sm.tolist())
        O.quantize_kv_write_paged(k.numpy(), v.numpy(), k_cache.numpy(), k_scale.numpy(), v_cache.numpy(),
                                  v_scale.numpy(), sm)

    rm.rotate_last = rotate_last
    lm.gaussian_codebook = lambda bits=3, block_size=128, device=None: torch.from_numpy(
        O.gaussian_codebook(bits, block_size))
    st.quantize_kv_write_paged = quantize_kv_write_paged
    st.quant, qm.rotation, qm.lloydmax = qm, rm, lm
    for name, mod in zip(STUB_NAMES, (st, qm, rm, lm)):
        sys.modules[name] = mod


def _load(root: Path, name: str):
    path = root / "superl8serve" / "engine" / "kv_cache.py"
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def trie_entries(cache) -> list:
    """Entries in the order ``_evict_one_prefix`` walks them (pre-order over
    children in insertion order): [token path, num_tokens, blocks, lru]."""
    out = []

    def walk(node, path):
        for k, v in node.items():
            if isinstance(k, str) and k.startswith("_"):
                continue
            if isinstance(v, dict):
                if "_entry" in v:
                    e = v["_entry"]
                    out.append([path + [k], e["num_tokens"], list(e["blocks"]), e["lru"]])
                walk(v, path + [k])

    walk(cache._prefix_trie, [])
    return out


def state(cache) -> dict:
    return {
        "free_blocks": list(cache._free_blocks),
        "free_slots": list(cache._free_slots),
        "slot_blocks": [list(b) for b in cache._slot_blocks],
        "refcount": sorted([int(k), int(v)] for k, v in cache._block_refcount.items()),
        "prefix_refs": sorted([int(k), int(v)] for k, v in cache._prefix_block_refs.items()),
        "entries": trie_entries(cache),
        "entry_count": cache._prefix_entry_count,
        "lru": cache._prefix_trie.get("_lru", 0),
        "used_blocks": cache.used_blocks,
        "pinned_prefix_blocks": cache.pinned_prefix_blocks,
        "prefix_block_bytes": cache.prefix_block_bytes(),
    }


TRACE_CONFIGS = [
    # (seed, ops, constructor kwargs)
    (1, 100, dict(num_slots=6, max_len=64, block_size=4, num_blocks=20)),
    (2, 100, dict(num_slots=6, max_len=64, block_size=4, num_blocks=24, max_prefix_entries=3)),
    (3, 100, dict(num_slots=5, max_len=32, block_size=2, num_blocks=16, max_prefix_blocks=3)),
    (4, 80, dict(num_slots=4, max_len=64, block_size=8, num_blocks=16, max_prefix_block_fraction=None)),
    (5, 100, dict(num_slots=6, max_len=48, block_size=4, num_blocks=18, max_prefix_entries=2, max_prefix_blocks=4)),
    # long prompts of 2-token blocks: one store adds several entries with one
    # LRU stamp, so the caps evict among tied entries
    (6, 100, dict(num_slots=6, max_len=32, block_size=2, num_blocks=48, max_prefix_entries=4)),
    (7, 100, dict(num_slots=6, max_len=32, block_size=2, num_blocks=48, max_prefix_blocks=5)),
]


def run_trace(mod, seed: int, n_ops: int, kw: dict) -> dict:
    rng = np.random.default_rng(seed)
    cache = mod.PagedKVCache(1, kw["num_slots"], 2, kw["max_len"], 32, device="cpu",
                             **{k: v for k, v in kw.items() if k not in ("num_slots", "max_len")})
    bs = kw["block_size"]
    bases = [rng.integers(0, 5, size=int(rng.integers(bs, 4 * bs + 1))).tolist() for _ in range(3)]
    live: dict[int, list[int]] = {}  # slot -> its tokens so far
    steps = []
    for _ in range(n_ops):
        r = rng.random()
        free_slots = list(cache._free_slots)
        if r < 0.16 or not live:
            op = {"op": "alloc"}
        elif r < 0.34:
            slot = int(rng.choice(sorted(live)))
            grow = int(rng.integers(1, 2 * bs + 1))
            op = {"op": "ensure_capacity", "slots": [slot], "lengths": [len(live[slot]) + grow], "grow": grow}
        elif r < 0.52:
            slot = int(rng.choice(sorted(live)))
            op = {"op": "store_prefix", "slot": slot, "tokens": list(live[slot])}
        elif r < 0.66:
            base = bases[int(rng.integers(len(bases)))]
            cut = int(rng.integers(0, len(base) + 1))
            toks = base[:cut] + rng.integers(0, 5, size=int(rng.integers(0, bs + 1))).tolist()
            op = {"op": "lookup_prefix", "tokens": toks}
            if free_slots and rng.random() < 0.6:
                op["then_share"] = True
        elif r < 0.8:
            slot = int(rng.choice(sorted(live)))
            op = {"op": "free", "slot": slot}
        else:
            slot = int(rng.choice(sorted(live)))
            base = bases[int(rng.integers(len(bases)))]
            op = {"op": "extend", "slot": slot, "tokens": base[: int(rng.integers(1, len(base) + 1))]}
        rec = dict(op)
        try:
            if op["op"] == "alloc":
                s = cache.alloc()
                live[s] = []
                rec["result"] = s
            elif op["op"] == "ensure_capacity":
                slot = op["slots"][0]
                cache.ensure_capacity(op["slots"], op["lengths"])
                live[slot] = live[slot] + rng.integers(0, 5, size=op["grow"]).tolist()
                rec["tokens_after"] = list(live[slot])
            elif op["op"] == "store_prefix":
                cache.store_prefix(op["tokens"], op["slot"])
            elif op["op"] == "lookup_prefix":
                n, blocks = cache.lookup_prefix(op["tokens"])
                rec["result"] = [n, list(blocks)]
                if op.get("then_share") and n > 0:
                    s = cache.alloc()
                    cache.share_blocks(s, blocks)
                    live[s] = list(op["tokens"][:n])
                    rec["shared_slot"] = s
            elif op["op"] == "free":
                cache.free(op["slot"])
                live.pop(op["slot"])
            elif op["op"] == "extend":  # grow the slot and give it these tokens (a prompt being written)
                slot = op["slot"]
                cache.ensure_capacity([slot], [len(op["tokens"])])
                live[slot] = list(op["tokens"]) if len(op["tokens"]) >= len(live[slot]) else live[slot]
                rec["tokens_after"] = list(live[slot])
        except RuntimeError as e:
            rec["error"] = str(e)
        rec["state"] = state(cache)
        steps.append(rec)
    return {"seed": seed, "config": kw, "steps": steps}


def eviction_functions(mod) -> dict:
    KV = mod.KVEviction
    out = {}
    out["block_bytes"] = [[h, b, d, vq, KV.block_bytes(h, b, d, v_quant=vq)]
                          for h in (1, 2, 8) for b in (4, 16, 256) for d in (32, 128, 256)
                          for vq in ("int8", "lloydmax3") if vq == "int8" or d % 128 == 0]
    out["adakv"] = [[n, t, lo, hi, KV.adakv_budgets(n, t, lo, hi)]
                    for n, t, lo, hi in ((1, 512, 128, 1024), (2, 512, 128, 1024), (12, 4096, 128, 1024),
                                         (24, 8192, 128, 1024), (36, 1000, 10, 100), (7, 3, 128, 1024),
                                         (4, 512, 64, 256), (5, 100000, 1, 1))]
    out["duoattn"] = [[h, f, *KV.duoattn_split(h, f)] for h in (1, 2, 8, 32, 40) for f in (0.0, 0.1, 0.25, 0.5, 1.0)]
    snap = []
    g = torch.Generator().manual_seed(7)
    for hq, hkv, d, seq, budget, layout in ((4, 2, 32, 24, 8, "2d"), (8, 2, 32, 16, 6, "2d"), (4, 4, 32, 40, 40, "4d"),
                                            (16, 4, 32, 96, 24, "4d"), (8, 8, 32, 64, 20, "2d"),
                                            (4, 1, 32, 10, 16, "2d")):
        # values on a 1/8 grid (short to store, exact in every float type);
        # the planted high-score keys differ from each other in one coordinate
        # so no two keys tie
        q = torch.randint(-12, 13, (hq, d), generator=g).float() / 8
        k = torch.randint(-12, 13, (hkv, seq, d), generator=g).float() / 8
        for i in range(seq // 3, min(seq, seq // 3 + budget // 2)):
            k[:, i] = q[0] * 2.0
            k[:, i, 0] += (i - seq // 3) / 8
        qa, ka = (q, k) if layout == "2d" else (q.reshape(1, hq, 1, d), k.unsqueeze(0))
        sel = KV.snapkv_selection(qa, ka, budget, hq, hkv)
        snap.append({"num_heads": hq, "num_kv_heads": hkv, "budget": budget, "layout": layout,
                     "q": q.numpy().tolist(), "k": k.numpy().tolist(), "selected": sel})
    out["snapkv"] = snap
    out["recall"] = []
    for a, b, t in (([1.0, 2.0, 3.0], [1.0, 2.0, 3.0], 0.99), ([1.0, 0.0, 0.0], [0.0, 1.0, 0.0], 0.99),
                    ([1.0, 2.0, 3.0], [1.0, 2.0, 3.1], 0.9999), ([0.5, -1.0], [0.5, -1.0], 1.0)):
        res = KV.recall_check(torch.tensor(a), torch.tensor(b), t)
        out["recall"].append({"a": a, "b": b, "threshold": t, "cos_sim": res["cos_sim"], "passed": res["passed"]})
    return out


COMPACT_CASES = [
    # (layers, slots, hkv, max_len, d, bs, seq_len, keep, extra allocations before)
    (2, 4, 2, 64, 32, 4, 8, list(range(8)), 0),
    (2, 4, 2, 64, 32, 4, 8, [0, 1, 2, 3], 0),
    (2, 4, 2, 128, 32, 8, 24, list(range(2, 14)), 1),
    (2, 4, 2, 64, 32, 8, 8, [], 0),
    (2, 2, 2, 64, 32, 4, 12, [0, 1, 2, 3], 1),
    (1, 3, 2, 128, 32, 4, 30, [1, 3, 5, 7, 9, 11, 13, 20, 29], 2),
    (3, 3, 1, 64, 32, 4, 16, [15], 0),
]


def compact_cases(mod, calls) -> list:
    out = []
    for layers, slots, hkv, max_len, d, bs, seq_len, keep, extra in COMPACT_CASES:
        cache = mod.PagedKVCache(layers, slots, hkv, max_len, d, device="cpu", block_size=bs)
        others = []
        for _ in range(extra):  # other slots interleave their blocks with the compacted one
            s = cache.alloc()
            cache.ensure_capacity([s], [bs + 1])
            others.append(s)
        slot = cache.alloc()
        cache.ensure_capacity([slot], [seq_len])
        g = torch.Generator().manual_seed(seq_len)
        for layer in range(layers):
            k = (torch.randn(1, hkv, seq_len, d, generator=g) * 0.1).half()
            v = (torch.randn(1, hkv, seq_len, d, generator=g) * 0.1).half()
            cache.write_prefill(layer, k, v, slot=slot)
        before = list(cache._slot_blocks[slot])
        free_before = list(cache._free_blocks)
        calls.clear()
        metrics = mod.KVEviction.compact(cache, slot, list(keep))
        out.append({"args": [layers, slots, hkv, max_len, d, bs, seq_len, keep, extra], "slot": slot,
                    "others": others, "blocks_before": before, "free_before": free_before,
                    "metrics": metrics, "blocks_after": list(cache._slot_blocks[slot]),
                    "free_after": list(cache._free_blocks),
                    "refcount_after": sorted([int(a), int(b)] for a, b in cache._block_refcount.items()),
                    "writes": [list(c) for c in calls]})
    return out


EVICT_CASES = [
    # (cfg kwargs, evict kwargs, layers, bs, seq_len, num_heads)
    (dict(enabled=False), dict(), 2, 8, 16, 4),
    (dict(enabled=True, policy="snapkv", kv_budget=8), dict(keep_mask=list(range(8))), 2, 4, 16, 4),
    (dict(enabled=True, policy="snapkv", kv_budget=8), dict(snap=True), 1, 4, 16, 4),
    (dict(enabled=True, kv_budget=4, recall_threshold=0.9999), dict(keep_mask=[0, 1, 2, 3], recall=([1.0, 0.0, 0.0], [0.0, 1.0, 0.0])), 1, 4, 8, 4),
    (dict(enabled=True, kv_budget=4, recall_threshold=0.99), dict(keep_mask=[0, 1, 2, 3], recall=([1.0, 2.0, 3.0], [1.0, 2.0, 3.0])), 1, 4, 8, 4),
    (dict(enabled=True, policy="adakv", kv_budget=512, adakv_min_budget=64, adakv_max_budget=256), dict(keep_mask=list(range(8))), 4, 4, 16, 4),
    (dict(enabled=True, policy="adakv", kv_budget=12, adakv_min_budget=2, adakv_max_budget=8), dict(), 4, 4, 16, 4),
    (dict(enabled=True, policy="adakv", kv_budget=12, adakv_min_budget=2, adakv_max_budget=8), dict(snap=True), 4, 4, 16, 4),
    (dict(enabled=True, policy="duoattn", kv_budget=8, duoattn_streaming_heads=0.25, duoattn_window=4), dict(keep_mask=list(range(8))), 2, 4, 16, 4),
    (dict(enabled=True, policy="duoattn", kv_budget=4, duoattn_window=4), dict(), 2, 4, 16, 4),
    (dict(enabled=True, policy="duoattn", kv_budget=4, duoattn_window=4), dict(snap=True), 2, 4, 16, 4),
    (dict(enabled=True, kv_budget=4), dict(keep_mask=[0, 1, 2, 3]), 2, 4, 12, 4),
    (dict(enabled=True, policy="other", kv_budget=5), dict(), 1, 4, 16, 4),
    (dict(enabled=True, kv_budget=32), dict(), 1, 4, 16, 4),
]


def evict_cases(mod) -> list:
    out = []
    for i, (cfg_kw, ev_kw, layers, bs, seq_len, nh) in enumerate(EVICT_CASES):
        hkv, d = 2, 32
        cache = mod.PagedKVCache(layers, 4, hkv, 64, d, device="cpu", block_size=bs)
        slot = cache.alloc()
        cache.ensure_capacity([slot], [seq_len])
        g = torch.Generator().manual_seed(100 + i)
        for layer in range(layers):
            k = (torch.randn(1, hkv, seq_len, d, generator=g) * 0.1).half()
            v = (torch.randn(1, hkv, seq_len, d, generator=g) * 0.1).half()
            cache.write_prefill(layer, k, v, slot=slot)
        kwargs = {}
        rec = {"config": cfg_kw, "layers": layers, "block_size": bs, "seq_len": seq_len, "num_heads": nh,
               "blocks_before": list(cache._slot_blocks[slot])}
        if "keep_mask" in ev_kw:
            kwargs["keep_mask"] = ev_kw["keep_mask"]
            rec["keep_mask"] = ev_kw["keep_mask"]
        if ev_kw.get("snap"):
            q = torch.randint(-12, 13, (nh, d), generator=g).float() / 8
            kf = torch.randint(-12, 13, (hkv, seq_len, d), generator=g).float() / 8
            for i in range(seq_len // 2):
                kf[:, i] = q[0] * 2.0
                kf[:, i, 0] += i / 8
            kwargs["q_last"], kwargs["k_full"] = q, kf
            rec["q_last"], rec["k_full"] = q.numpy().tolist(), kf.numpy().tolist()
        if "recall" in ev_kw:
            full, after = ev_kw["recall"]
            kwargs["logits_full"] = torch.tensor(full)
            kwargs["logits_fn"] = lambda a=after: torch.tensor(a)
            rec["logits_full"], rec["logits_after"] = full, after
        res = cache.evict_after_prefill(slot, seq_len, eviction_config=mod.EvictionConfig(**cfg_kw), num_heads=nh,
                                        **kwargs)
        rec["result"] = res
        rec["blocks_after"] = list(cache._slot_blocks[slot])
        rec["free_after"] = list(cache._free_blocks)
        out.append(rec)
    return out


def shim_import(root: Path) -> dict:
    """Load the module again with this repository's superl8 interface as
    ``superl8`` (no kernel runs: import only)."""
    for name in STUB_NAMES:
        sys.modules.pop(name, None)
    from superl8_serve_amd import shim

    pkg = shim.install()
    mod = _load(root, "ref_kv_cache_with_shim")
    from superl8_serve_amd.superl8.quant import rotation

    return {"imported": True, "superl8_is_shim": mod.superl8 is pkg,
            "rotate_last_is_shim": mod.rotate_last is rotation.rotate_last}


def main() -> None:
    root = Path(sys.argv[1]) if len(sys.argv) > 1 else Path("/root/reference")
    calls: list = []
    _install_cpu_stub(calls)
    mod = _load(root, "ref_kv_cache")
    data = {
        "source": "superl8serve/engine/kv_cache.py",
        "traces": [run_trace(mod, seed, n, kw) for seed, n, kw in TRACE_CONFIGS],
        **eviction_functions(mod),
        "compact": compact_cases(mod, calls),
        "evict": evict_cases(mod),
        "shim_import": shim_import(root),
    }
    OUT.write_text(json.dumps(data, separators=(",", ":")) + "\n")
    print(f"wrote {OUT} ({OUT.stat().st_size // 1024} KiB)")


if __name__ == "__main__":
    main()
