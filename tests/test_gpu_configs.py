"""GPU parity at the benchmark workloads themselves (one layer each), through
the C ABI, against the oracle:

* Qwen3-8B int8 decode step, batch 64, lognormal contexts up to 8192 (the
  headline workload, default stream-K slicing, append in the decode launch);
* Qwen3-8B K8V3 decode step, batch 32, contexts U{8192..32768};
* chunked prefill with prefix caching: 16 sequences share a 4096-token prefix
  held in refcounted blocks, each copies its last shared block on write,
  appends a 512-token chunk and attends causally; then 20 % of the blocks are
  freed and the pool is compacted;
* tree verify, batch 32, 8192-token prefixes, random trees of 16-64 nodes.

The inputs are the benchmark's own generators (``bench.py``).  Cache bytes
are compared bit for bit: the appended tokens in full, the prefix of a
seeded subset of rows (the oracle's append is ~0.2 ms per token on the
host).  Attention outputs are compared with the float64 oracle over the
dequantized cache: every row of every workload.  Each comparison prints the
plain max-abs error beside the scaled one the tolerance is stated in
(``max |out - ref| / max(1, |ref|)``: an fp16 output holds ~11 significant
bits, so above |ref| = 1 the bound is relative)."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import bench
from oracle import kv_oracle as O
from superl8_serve_amd import ops
from superl8_serve_amd.paged_cache import PagedKVCache

pytestmark = pytest.mark.gpu

DEV = "cuda"
SCALE = 1.0 / math.sqrt(bench.D)


def _np(t):
    return t.detach().cpu().numpy()


def _same(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def _rows_of(slots):
    return O.flat_rows(np.asarray(slots), bench.HKV, bench.BS).reshape(-1)


def _check_int8_rows(cache, k, v, slots, what):
    """The storage rows of `slots` hold the oracle's int8 append of k, v."""
    kc, ks, vc, vs = cache
    kq, kscale = O.quantize_i8_rowwise(O.rotate_last(np.asarray(k, np.float16)))
    vq, vscale = O.quantize_i8_rowwise(np.asarray(v, np.float16))
    rows = _rows_of(slots)
    d = bench.D
    assert _same(kc.reshape(-1, d)[rows], kq.reshape(-1, d)), f"{what}: K codes differ from the oracle"
    assert _same(ks.reshape(-1)[rows], kscale.reshape(-1)), f"{what}: K scales differ from the oracle"
    assert _same(vc.reshape(-1, d)[rows], vq.reshape(-1, d)), f"{what}: V codes differ from the oracle"
    assert _same(vs.reshape(-1)[rows], vscale.reshape(-1)), f"{what}: V scales differ from the oracle"


def _check_k8v3_rows(cache, k, v, slots, codebook, what):
    kc, ks, vp, vn = cache
    ref = [np.zeros_like(x) for x in cache]
    O.k8v3_write_paged(np.asarray(k, np.float16), np.asarray(v, np.float16), *ref, codebook, slots)
    rows = _rows_of(slots)
    n_rows = kc.shape[0] * kc.shape[1] * kc.shape[2]
    for got, want, name in zip(cache, ref, ("K codes", "K scales", "V words", "V norms")):
        g, w = got.reshape(n_rows, -1), want.reshape(n_rows, -1)
        assert _same(g[rows], w[rows]), f"{what}: {name} differ from the oracle"


def _assert_close(got, ref, what):
    """Tolerance against the float64 oracle, reporting the plain max-abs
    error as well as the scaled one the bound applies to."""
    mx, rel = O.attention_errors(got, ref)
    plain = float(np.max(np.abs(np.asarray(got, np.float64) - ref))) if ref.size else 0.0
    print(f"{what}: scaled max err {mx:.3e} (plain max-abs {plain:.3e}, max |ref| {np.abs(ref).max():.2f}), "
          f"rel rms {rel:.3e}", flush=True)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"


def _unchanged_except(before, after, rows, what):
    """Every storage row but `rows` is byte-identical."""
    for b, a, name in zip(before, after, ("k_cache", "k_scale", "v_cache", "v_scale")):
        b2 = b.reshape(b.shape[0] * b.shape[1] * b.shape[2], -1)
        a2 = a.reshape(b2.shape)
        keep = np.ones(b2.shape[0], bool)
        keep[rows] = False
        assert _same(a2[keep], b2[keep]), f"{what}: {name} changed outside the appended rows"


def test_c2_int8_decode_step_batch64():
    """The headline step, one layer: append + decode in one launch at the
    default slicing.  Prefix bytes of 8 seeded rows, every appended byte and
    every row's attention against the oracle; output bit-identical to the
    reference's two calls (append kernel, then decode)."""
    print("C2: building the batch-64 workload (1 layer)", flush=True)
    w = bench.build(DEV, layers=1, keep_prefix=True)
    lens, bt = w["lens"], w["bt_np"]
    pre = [_np(w[k][0]) for k in ("kc", "ks", "vc", "vs")]
    # prefix append: the tokens of 8 seeded rows
    rng = np.random.default_rng(21)
    starts = np.concatenate([[0], np.cumsum(lens - 1)])
    kp, vp = (_np(x) for x in w["prefix"][0])
    for b in rng.choice(bench.BATCH, 8, replace=False):
        sl = slice(int(starts[b]), int(starts[b + 1]))
        _check_int8_rows(pre, kp[sl], vp[sl], w["pre_slots"][sl], f"C2 prefix of row {b}")
    del kp, vp, w["prefix"][:]

    # the reference's two calls on a copy of the cache
    sep = [torch.from_numpy(x).to(DEV) for x in pre]
    ops.quantize_kv_write_paged(w["k_new"][0], w["v_new"][0], *sep, w["new_sm"])
    want = ops.attn_paged_decode_cached(w["q"][0], *sep, w["bt"], w["cl"], bench.BS,
                                        max_context_len=bench.MAX_LEN, scale=SCALE)
    print("C2: one-launch decode step", flush=True)
    got = bench.decode_layer(w, 0, fused=True)
    torch.cuda.synchronize()
    after = [_np(w[k][0]) for k in ("kc", "ks", "vc", "vs")]
    assert _same(_np(got), _np(want)), "C2: one-launch output differs from append + decode"
    for a, s, name in zip(after, sep, ("k_cache", "k_scale", "v_cache", "v_scale")):
        assert _same(a, _np(s)), f"C2: {name} differs from the append kernel's"
    _check_int8_rows(after, _np(w["k_new"][0]), _np(w["v_new"][0]), w["new_slots"], "C2 appended tokens")
    _unchanged_except(pre, after, _rows_of(w["new_slots"]), "C2")
    print("C2: oracle attention over all 64 rows", flush=True)
    ref = O.paged_decode(_np(w["q"][0])[:, :, 0, :], O.LayerCache(*after), bt, lens, SCALE)
    _assert_close(_np(got.float())[:, :, 0, :], ref, "C2 (64 rows)")


def test_c3_k8v3_decode_step_batch32_long_context():
    """K8V3 step, one layer: every appended token bit-exact, the first 2048
    prefix tokens of 2 seeded rows bit-exact, one launch == append kernel +
    K8V3 decode for all 32 rows, and all 32 rows against the oracle."""
    rng = np.random.default_rng(31)
    keep = tuple(int(x) for x in rng.choice(bench.K8V3_BATCH, 2, replace=False))
    print(f"C3: building the batch-32 K8V3 workload (1 layer), prefix rows {keep}", flush=True)
    w = bench.k8v3_workload(DEV, layers=1, keep_rows=keep)
    lens, bt, cb = w["lens"], w["bt_np"], _np(w["cb"])
    pre = [_np(w[k][0]) for k in ("kc", "ks", "vp", "vn")]
    for b, c0, kp, vq in w["prefix_kv"]:
        n = min(2048, kp.shape[0])
        p_ = np.arange(c0, c0 + n)
        slots = (bt[b, p_ // bench.BS] * bench.BS + p_ % bench.BS).astype(np.int32)
        _check_k8v3_rows(pre, _np(kp[:n]), _np(vq[:n]), slots, cb, f"C3 prefix of row {b}")
    w["prefix_kv"].clear()

    sep = [torch.from_numpy(x).to(DEV) for x in pre]
    ops.quantize_kv_write_paged_k8v3(w["k_new"][0], w["v_new"][0], *sep, w["cb"], w["new_sm"])
    want = ops.attn_paged_decode_k8v3(w["q"][0], *sep, w["cb"], w["bt"], w["cl"], bench.BS,
                                      max_context_len=w["max_ctx"], scale=SCALE)
    print("C3: one-launch K8V3 decode step", flush=True)
    got = ops.attn_paged_decode_append_k8v3(w["q"][0], w["k_new"][0], w["v_new"][0], w["kc"][0], w["ks"][0],
                                            w["vp"][0], w["vn"][0], w["cb"], w["bt"], w["cl"], bench.BS,
                                            max_context_len=w["max_ctx"], scale=SCALE)
    torch.cuda.synchronize()
    after = [_np(w[k][0]) for k in ("kc", "ks", "vp", "vn")]
    assert _same(_np(got), _np(want)), "C3: one-launch output differs from append + decode"
    for a, s, name in zip(after, sep, ("k_cache", "k_scale", "v_packed", "v_norm")):
        assert _same(a, _np(s)), f"C3: {name} differs from the append kernel's"
    _check_k8v3_rows(after, _np(w["k_new"][0]), _np(w["v_new"][0]), w["new_slots"], cb, "C3 appended tokens")
    _unchanged_except(pre, after, _rows_of(w["new_slots"]), "C3")
    print("C3: oracle attention over all 32 rows", flush=True)
    layer = O.LayerCache(after[0], after[1], v_packed=after[2], v_norm=after[3], v_codebook=cb)
    ref = O.paged_decode(_np(w["q"][0])[:, :, 0, :], layer, bt, lens, SCALE)
    _assert_close(_np(got.float())[:, :, 0, :], ref, "C3 (32 rows)")


def _fp16(gen, shape, ch):
    x = torch.randn(shape, generator=gen, device=DEV, dtype=torch.float32)
    x[..., ch] *= bench.OUTLIER_SCALE
    return x.half()


def test_c4_chunked_prefill_prefix_cow_and_compaction():
    """16 sequences share a 4096-token prefix through the prefix cache;
    each copies its last shared block on write, appends a 512-token chunk and
    attends causally over 4608 keys; then a seeded 20 % of the blocks is freed
    and the pool compacted.  Checks: chunk bytes, the copy, all 16
    sequences' attention against the oracle, every read_dense and every
    sequence's attention unchanged by the compaction, the live blocks packed
    at the bottom of the pool."""
    hkv, d, bs, hq = bench.HKV, bench.D, bench.BS, bench.HQ
    prefix_len, chunk, nseq = 4096, 512, 16
    gen = torch.Generator(device=DEV).manual_seed(3)
    rng = np.random.default_rng(3)
    ch = torch.from_numpy(rng.choice(d, bench.OUTLIER_CH, replace=False)).to(DEV)
    cache = PagedKVCache(1, nseq + 1, hkv, prefix_len + chunk, d, device=DEV, block_size=bs)
    owner = cache.alloc()
    cache.ensure_capacity([owner], [prefix_len])
    kp, vp = _fp16(gen, (1, hkv, prefix_len, d), ch), _fp16(gen, (1, hkv, prefix_len, d), ch)
    cache.write_prefill(0, kp, vp, slot=owner)
    tokens = rng.integers(0, 150000, size=prefix_len).tolist()
    cache.store_prefix(tokens, owner)
    slots, chunks = [], []
    print("C4: prefix shared by 16 sequences, copy-on-write, 512-token chunks", flush=True)
    for i in range(nseq):
        s = cache.alloc()
        n, blocks = cache.lookup_prefix(tokens + [int(x) for x in rng.integers(0, 150000, size=chunk)])
        assert n == prefix_len and len(blocks) == prefix_len // bs
        cache.share_blocks(s, blocks)
        last = blocks[-1]
        refs = cache._block_refcount[last]
        new = cache.copy_on_write_last_block(s)
        assert new is not None and cache._block_refcount[last] == refs - 1 and cache._slot_blocks[s][-1] == new
        cache.ensure_capacity([s], [prefix_len + chunk])
        kc_, vc_ = _fp16(gen, (1, hkv, chunk, d), ch), _fp16(gen, (1, hkv, chunk, d), ch)
        pos = torch.arange(prefix_len, prefix_len + chunk, device=DEV)
        cache.write_prefill(0, kc_, vc_, slot=s, positions=pos)
        slots.append(s)
        chunks.append((kc_, vc_))
    torch.cuda.synchronize()
    pool = [_np(t[0]) for t in cache._tensors()]
    # the copies hold the shared block's bytes
    shared_last = cache._slot_blocks[owner][-1]
    for s in slots:
        blk = cache._slot_blocks[s][prefix_len // bs - 1]
        for t in pool:
            assert _same(t[blk], t[shared_last]), "C4: copy-on-write block differs from its source"
    # chunk bytes
    for s, (kc_, vc_) in zip(slots, chunks):
        sm = cache.flat_slot_mapping(s, prefix_len + chunk)[prefix_len:]
        _check_int8_rows(pool, _np(kc_[0].transpose(0, 1)), _np(vc_[0].transpose(0, 1)), sm, f"C4 chunk of slot {s}")

    q = _fp16(gen, (nseq, chunk, hq, d), ch).transpose(1, 2)  # [B, Hq, S, D] view, as the layer passes it
    print("C4: chunked-prefill attention (16 x 512 queries over 4608 keys)", flush=True)
    out = cache.verify_attn(0, q, slots, [prefix_len] * nseq, scale=SCALE)
    torch.cuda.synchronize()
    bt = _np(cache.block_table(slots))
    rng.choice(nseq, 3, replace=False)  # (keeps the seeded draws below unchanged)
    print("C4: oracle attention of all 16 sequences", flush=True)
    ref = O.paged_verify(_np(q), O.LayerCache(*pool), bt, np.full(nseq, prefix_len), SCALE)
    _assert_close(_np(out.float()), ref, "C4 (16 sequences)")

    # free a seeded 20 % of the allocated blocks (whole sequences: 3 private
    # blocks each), then compact the pool
    used0 = cache.used_blocks
    victims = []
    for s in rng.permutation(slots):
        if 3 * len(victims) >= 0.2 * used0:
            break
        victims.append(int(s))
    live = [s for s in slots if s not in victims]
    length = {s: prefix_len + chunk for s in live}
    length[owner] = prefix_len
    dense = {s: [_np(x) for x in cache.read_dense(0, s, n)] for s, n in length.items()}
    out_live = _np(cache.verify_attn(0, q[[slots.index(s) for s in live]], live, [prefix_len] * len(live),
                                     scale=SCALE))
    for s in victims:
        cache.free(s)
    print(f"C4: freed {len(victims)} sequences ({used0 - cache.used_blocks} blocks), compacting", flush=True)
    before = [_np(t[0]) for t in cache._tensors()]
    moves = cache.defragment()
    torch.cuda.synchronize()
    assert moves, "C4: nothing to compact"
    after = [_np(t[0]) for t in cache._tensors()]
    want = [x.copy() for x in before]
    O.copy_blocks([x[None] for x in want], [m[0] for m in moves], [m[1] for m in moves])
    for a, b in zip(after, want):
        assert _same(a, b), "C4: compaction moved bytes other than the oracle's block copy"
    held = {blk for s in live + [owner] for blk in cache._slot_blocks[s]}
    assert held <= set(range(cache.used_blocks)), "C4: live blocks not packed at the bottom of the pool"
    for s, n in length.items():
        k2, v2 = (_np(x) for x in cache.read_dense(0, s, n))
        assert _same(k2, dense[s][0]) and _same(v2, dense[s][1]), f"C4: read_dense of slot {s} changed"
    out2 = _np(cache.verify_attn(0, q[[slots.index(s) for s in live]], live, [prefix_len] * len(live), scale=SCALE))
    assert _same(out2, out_live), "C4: attention changed by the compaction"
    n, blocks = cache.lookup_prefix(tokens)
    assert n == prefix_len and blocks == cache._slot_blocks[owner][: prefix_len // bs]


@pytest.mark.parametrize("k8v3", [False, True], ids=["int8", "k8v3"])
def test_c5_tree_verify_batch32(k8v3):
    """32 sequences with 8192-token prefixes append random draft trees of
    16-64 nodes (branching 1-4) and attend prefix + ancestors: appended bytes
    bit-exact, all 32 rows against the oracle."""
    print(f"C5: building the tree-verify workload ({'k8v3' if k8v3 else 'int8'}, 1 layer)", flush=True)
    w, info = bench.verify_workload("tree", DEV, k8v3=k8v3, layers=1)
    before = [_np(w[k][0]) for k in ("kc", "ks", "vc", "vs")]
    w["append"](w["k_new"][0], w["v_new"][0], 0, w["new_sm"])
    kw = dict(query_lens=w["ql"], tree_mask=w["tree"], max_context_len=w["max_ctx"], scale=SCALE)
    if k8v3:
        out = ops.attn_paged_verify_k8v3(w["q"][0], w["kc"][0], w["ks"][0], w["vc"][0], w["vs"][0], w["cb"],
                                         w["bt"], w["prefix"], bench.BS, **kw)
    else:
        out = ops.attn_paged_verify(w["q"][0], w["kc"][0], w["ks"][0], w["vc"][0], w["vs"][0], w["bt"],
                                    w["prefix"], bench.BS, **kw)
    torch.cuda.synchronize()
    after = [_np(w[k][0]) for k in ("kc", "ks", "vc", "vs")]
    kn, vn = _np(w["k_new"][0]), _np(w["v_new"][0])
    if k8v3:
        _check_k8v3_rows(after, kn, vn, w["new_slots"], _np(w["cb"]), "C5 drafts")
    else:
        _check_int8_rows(after, kn, vn, w["new_slots"], "C5 drafts")
    _unchanged_except(before, after, _rows_of(w["new_slots"]), "C5")
    rows = np.arange(info["batch"])
    print("C5: oracle attention over all 32 rows", flush=True)
    if k8v3:
        layer = O.LayerCache(after[0], after[1], v_packed=after[2], v_norm=after[3], v_codebook=_np(w["cb"]))
    else:
        layer = O.LayerCache(*after)
    ref = O.paged_verify(_np(w["q"][0])[rows], layer, w["bt_np"][rows], w["prefix_np"][rows],
                         SCALE, query_lens=w["nq_np"][rows], tree_mask=w["tree_np"][rows])
    got = _np(out.float())[rows]
    for i, r in enumerate(rows):  # queries past a row's node count are zeros
        assert not got[i, :, w["nq_np"][r]:].any()
    _assert_close(got, ref, f"C5 {'k8v3' if k8v3 else 'int8'} (32 rows)")
