"""GPU parity of the verify's key-range split against the oracle, through the
C ABI: each (sequence, KV head, query block) split across workgroups whose
partials a second kernel combines.  The split is taken when a call has fewer
units than the GPU keeps resident (batch-1 speculative decoding) or more than
2^20 keys per unit; s8kv_verify_set_splits forces a count here, including counts
that leave splits without keys."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import _lib, ops
from tests.kvcase import make_case
from tests.kvgpu import CODEBOOK, alloc, append, assert_close, layer, t, to_np, verify

pytestmark = pytest.mark.gpu


@pytest.fixture
def force_splits():
    """Set the verify's split count (0: planned per call); reset on exit."""
    lib = _lib.load()

    def set_(n):
        _lib.check(lib.s8kv_verify_set_splits(int(n)), "s8kv_verify_set_splits")

    yield set_
    set_(0)


def _random_tree(rng, n):
    """Ancestor bit masks of a random tree over n drafts (node i's parent < i)."""
    masks = np.zeros(n, np.int64)
    for i in range(n):
        par = int(rng.integers(-1, i)) if i else -1
        masks[i] = (masks[par] if par >= 0 else 0) | (1 << i)
    return masks


def _case(seed, kind, hq, hkv, d, bs, prefix, nq):
    prefix = np.asarray(prefix)
    case = make_case(seed, len(prefix), hq, hkv, d, bs, prefix + nq, outlier_channels=2 if d >= 128 else 0)
    cache = alloc(kind, case.num_blocks, hkv, bs, d)
    append(kind, t(case.k), t(case.v), cache, t(case.slots))
    qv = np.random.default_rng(seed + 1).standard_normal((len(prefix), hq, nq, d)).astype(np.float16)
    return case, cache, tuple(to_np(x) for x in cache), qv, prefix


def _run(kind, case, cache, qv, prefix, tree_mask=None, window=None, query_lens=None):
    fn = ops.attn_paged_verify if kind == "int8" else ops.attn_paged_verify_k8v3
    extra = () if kind == "int8" else (t(CODEBOOK),)
    out = fn(t(qv), *cache, *extra, t(case.block_table), t(prefix.astype(np.int32)), case.block_size,
             query_lens=None if query_lens is None else t(np.asarray(query_lens, np.int32)),
             tree_mask=None if tree_mask is None else t(tree_mask), max_context_len=int(case.lens.max()),
             scale=case.scale, window=window)
    torch.cuda.synchronize()
    return to_np(out.float())


@pytest.mark.parametrize("kind,d,splits", [
    ("int8", 128, 5), ("int8", 64, 3), ("int8", 256, 9), ("k8v3", 128, 7), ("k8v3", 256, 4),
])
def test_forced_split_matches_oracle_and_unsplit(kind, d, splits, force_splits):
    case, cache, host, qv, prefix = _case(900 + d + splits, kind, 8, 2, d, 16, [3000, 517, 40], 6)
    ref = O.paged_verify(qv, layer(kind, host), case.block_table, prefix, case.scale)
    force_splits("1")
    whole = _run(kind, case, cache, qv, prefix)
    assert_close(whole, ref, f"{kind} D={d} unsplit")
    force_splits(str(splits))
    split = _run(kind, case, cache, qv, prefix)
    assert_close(split, ref, f"{kind} D={d} {splits} splits")
    assert_close(split, whole.astype(np.float64), f"{kind} D={d} {splits} splits vs unsplit")


@pytest.mark.parametrize("splits", [2, 31, 200])
def test_split_tree_and_empty_splits(splits, force_splits):
    """Tree masks across splits; 200 splits of a few hundred keys leave most
    splits of the short rows without keys."""
    nq = 12
    case, cache, host, qv, prefix = _case(950 + splits, "int8", 16, 4, 128, 32, [4096, 33, 0, 700], nq)
    rng = np.random.default_rng(951)
    tm = np.stack([_random_tree(rng, nq) for _ in range(len(prefix))])
    force_splits(str(splits))
    got = _run("int8", case, cache, qv, prefix, tree_mask=tm)
    ref = O.paged_verify(qv, layer("int8", host), case.block_table, prefix, case.scale, tree_mask=tm)
    assert_close(got, ref, f"tree verify, {splits} splits")


@pytest.mark.parametrize("kind,splits", [("int8", 4), ("int8", 1), ("k8v3", 7)])
def test_split_query_lens(kind, splits, force_splits):
    """Rows past a sequence's query count are zeros also when they share a
    query block with live rows (G 4: positions 0-15 per 64-row block) and
    the block's keys are split; the live rows match the oracle."""
    nq = 24
    ql = np.array([5, 24, 0, 17])
    case, cache, host, qv, prefix = _case(990 + splits, kind, 16, 4, 128, 32, [3000, 2100, 1500, 2600], nq)
    force_splits(str(splits))
    got = _run(kind, case, cache, qv, prefix, query_lens=ql)
    ref = O.paged_verify(qv, layer(kind, host), case.block_table, prefix, case.scale, query_lens=ql)
    for b, n in enumerate(ql):
        assert not got[b, :, n:].any(), f"row {b}: outputs past its {n} queries"
    assert_close(got, ref, f"{kind} verify with query_lens, {splits} splits")


@pytest.mark.parametrize("kind", ["int8", "k8v3"])
def test_split_window_verify(kind, force_splits):
    case, cache, host, qv, prefix = _case(960, kind, 8, 2, 128, 16, [5000, 300], 5)
    force_splits("6")
    got = _run(kind, case, cache, qv, prefix, window=1024)
    ref = O.paged_verify(qv, layer(kind, host), case.block_table, prefix, case.scale, window=1024)
    assert_close(got, ref, f"{kind} window verify, 6 splits")


@pytest.mark.parametrize("kind", ["int8", "k8v3"])
def test_split_window_verify_with_fresh_drafts(kind, force_splits):
    """A window verify whose drafts come fresh (fp16 K / V rows, not the
    cache's) split into 5 key ranges: the drafts' tiles sit in the last
    ranges, and the result matches the oracle in that mode."""
    nq = 37
    case, cache, host, qv, prefix = _case(965, kind, 16, 4, 128, 16, [4000, 700], nq)
    starts = np.concatenate([[0], np.cumsum(case.lens)])
    idx = np.stack([starts[b] + prefix[b] + np.arange(nq) for b in range(len(prefix))])
    kd, vd = case.k[idx], case.v[idx]
    force_splits("5")
    fn = ops.attn_paged_verify if kind == "int8" else ops.attn_paged_verify_k8v3
    extra = () if kind == "int8" else (t(CODEBOOK),)
    out = fn(t(qv), *cache, *extra, t(case.block_table), t(prefix.astype(np.int32)), case.block_size,
             max_context_len=int(case.lens.max()), scale=case.scale, window=900, k_draft=t(kd), v_draft=t(vd))
    torch.cuda.synchronize()
    ref = O.paged_verify(qv, layer(kind, host), case.block_table, prefix, case.scale, window=900,
                         fresh_drafts=(kd, vd))
    assert_close(to_np(out.float()), ref, f"{kind} window verify with fresh drafts, 5 splits")


@pytest.mark.parametrize("kind", ["int8", "k8v3"])
def test_batch_one_long_context_plans_a_split(kind):
    """Batch 1 with a 32K prefix and a 32-node tree at Qwen3-8B heads has 8
    units (one 128-row query block per KV head): the default plan splits
    each into 64 key ranges of 512 keys within the workspace the size query
    gives, and the combined result matches the oracle."""
    nq = 32
    ws = _lib.load().s8kv_verify_workspace_size(1, 32, 8, 128, nq, 32768 + nq)
    assert ws > 0
    case, cache, host, qv, prefix = _case(970, kind, 32, 8, 128, 256, [32768], nq)
    tm = _random_tree(np.random.default_rng(971), nq)[None]
    got = _run(kind, case, cache, qv, prefix, tree_mask=tm)
    ref = O.paged_verify(qv, layer(kind, host), case.block_table, prefix, case.scale, tree_mask=tm)
    assert_close(got, ref, f"{kind} batch-1 tree verify (planned split)")


def test_split_graph_replays(force_splits):
    """Both launches of a split verify captured in a HIP graph: every replay
    returns the eager result."""
    force_splits("8")
    case, cache, host, qv, prefix = _case(980, "int8", 8, 2, 128, 16, [2000, 900], 4)
    eager = _run("int8", case, cache, qv, prefix)
    q, bt, pl = t(qv), t(case.block_table), t(prefix.astype(np.int32))
    mc = int(case.lens.max())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.attn_paged_verify(q, *cache, bt, pl, case.block_size, max_context_len=mc, scale=case.scale)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.attn_paged_verify(q, *cache, bt, pl, case.block_size, max_context_len=mc, scale=case.scale)
    for _ in range(3):
        torch.zeros(1 << 20, device="cuda").add_(1.0)  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(to_np(out.float()), eager)
