"""GPU tests of the per-step slice plan (``attn_paged_decode_plan`` and the
``plan=`` form of the one-launch decode step ops).

A planned launch reads, from the plan, what the unplanned launch computes in
its prologue (the slice of the token stream each workgroup takes, the
segment it processes first, and the storage rows of its waves' first tiles),
so its cache bytes and outputs must equal the unplanned launch's bit for bit,
for every slicing.  A plan made for other buffers or another geometry must be
ignored, and the plan's entries must tile the token stream."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import empty_int8_cache, empty_k8v3_cache, make_case

pytestmark = pytest.mark.gpu

DEV = "cuda"
CODEBOOK = O.gaussian_codebook(3, 128)
HEADER, ENTRY = 32, 16  # plan words: header, then one entry per workgroup column


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _np(t):
    return t.detach().cpu().numpy()


def _last_tokens(case):
    """The cache without each row's last token (oracle append), the rows' last
    tokens [B, Hkv, D] (zeros for empty rows)."""
    ends = np.cumsum(case.lens)
    last = ends - 1
    has = case.lens > 0
    keep = np.ones(int(ends[-1]) if len(ends) else 0, bool)
    keep[last[has]] = False
    k_new = np.zeros((case.batch, case.num_kv_heads, case.head_dim), np.float16)
    v_new = np.zeros_like(k_new)
    k_new[has] = case.k[last[has]]
    v_new[has] = case.v[last[has]]
    return keep, k_new, v_new


class _Step:
    """One layer's fused decode step over device copies of a case, run with
    and without a plan on the same block-table and length tensors."""

    def __init__(self, case, layout):
        self.case, self.layout = case, layout
        keep, k_new, v_new = _last_tokens(case)
        if layout == "int8":
            self.pre = empty_int8_cache(case)
            O.quantize_kv_write_paged(case.k[keep], case.v[keep], *self.pre, case.slots[keep])
        else:
            self.pre = empty_k8v3_cache(case)
            O.k8v3_write_paged(case.k[keep], case.v[keep], *self.pre, CODEBOOK, case.slots[keep])
        self.kn, self.vn = _t(k_new), _t(v_new)
        self.q = _t(case.q)[:, :, None, :]
        self.bt = _t(case.block_table)
        self.cl = _t(case.lens.astype(np.int32))
        self.cb = _t(CODEBOOK)
        self.max_ctx = int(case.lens.max())

    def plan(self, **kw):
        kw.setdefault("max_context_len", self.max_ctx)
        return ops.attn_paged_decode_plan(_t(self.pre[0]), kw.pop("bt", self.bt), kw.pop("cl", self.cl),
                                          self.case.block_size, num_q_heads=self.case.num_q_heads,
                                          layout=self.layout, **kw)

    def run(self, plan=None, cache=None):
        c = self.case
        cache = [_t(x) for x in self.pre] if cache is None else cache
        if self.layout == "int8":
            out = ops.attn_paged_decode_append(self.q, self.kn, self.vn, *cache, self.bt, self.cl, c.block_size,
                                               max_context_len=self.max_ctx, scale=c.scale, plan=plan)
        else:
            kc, ks, vp, vnrm = cache
            out = ops.attn_paged_decode_append_k8v3(self.q, self.kn, self.vn, kc, ks, vp, vnrm, self.cb, self.bt,
                                                    self.cl, c.block_size, max_context_len=self.max_ctx,
                                                    scale=c.scale, plan=plan)
        torch.cuda.synchronize()
        return _np(out.float()), [_np(x) for x in cache]


def _same(a, b, what):
    out_a, cache_a = a
    out_b, cache_b = b
    for x, y, name in zip(cache_a, cache_b, ("k_cache", "k_scale", "v", "v_scale")):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"{what}: {name} differs"
    assert np.array_equal(out_a, out_b), f"{what}: outputs differ (max {np.abs(out_a - out_b).max():.3e})"


@pytest.mark.parametrize("layout,hq,hkv,d,bs,lens", [
    ("int8", 32, 8, 128, 256, "qwen"),                 # Qwen3-8B heads, ragged lengths
    ("int8", 16, 8, 128, 16, [100, 17, 16, 15, 1, 0]),  # block_size < 32: no first tile in the plan
    ("int8", 16, 8, 128, 256, [256, 257, 512, 255]),
    ("int8", 8, 2, 256, 32, [50, 129, 4000]),
    ("int8", 8, 4, 64, 64, [33, 2, 80, 0, 700]),
    ("int8", 4, 2, 32, 32, "many"),                    # more than 64 rows (the scans' second pass)
    ("k8v3", 32, 8, 128, 256, "long"),
    ("k8v3", 8, 2, 256, 32, [50, 129, 300, 2100]),
])
def test_planned_step_equals_unplanned(layout, hq, hkv, d, bs, lens):
    rng = np.random.default_rng(11)
    if lens == "qwen":
        lens = rng.integers(200, 3000, size=16).tolist()
    elif lens == "long":
        lens = rng.integers(1500, 6000, size=8).tolist()
    elif lens == "many":
        lens = rng.integers(0, 300, size=100).tolist()
    case = make_case(4100 + hq + d + bs, len(lens), hq, hkv, d, bs, lens, outlier_channels=2 if d == 128 else 0)
    step = _Step(case, layout)
    plan = step.plan()
    _same(step.run(plan), step.run(None), f"{layout} planned")


@pytest.mark.parametrize("wg_per_head,ghost,batch,bs,lens", [
    (1, 128, 4, 32, [1000, 129, 5000, 0]),          # one slice per head, rows past 2048 tokens
    (2, 0, 4, 256, [5000, 100, 0, 37]),             # a split row's later block-id stage
    (7, 0, 64, 32, "short"),                        # rows split across slices, reordered segments
    (40, 512, 64, 32, "short"),                     # slices holding no tokens
    (3, 64, 5, 8, [300, 1, 64, 2500, 31]),          # block_size < 32
])
def test_planned_step_slicings(wg_per_head, ghost, batch, bs, lens, monkeypatch):
    monkeypatch.setenv("S8KV_DECODE_WG_PER_HEAD", str(wg_per_head))
    monkeypatch.setenv("S8KV_DECODE_GHOST", str(ghost))
    if lens == "short":
        lens = np.random.default_rng(6).integers(0, 120, size=batch).tolist()
    case = make_case(177 + wg_per_head, batch, 32, 8, 128, bs, lens)
    step = _Step(case, "int8")
    _same(step.run(step.plan()), step.run(None), f"planned wg/head={wg_per_head}")


def test_plan_for_other_buffers_or_geometry_is_ignored():
    """A plan names the block table, lengths and geometry it was made for; a
    launch given a plan for anything else locates its work itself."""
    case = make_case(4242, 12, 32, 8, 128, 256, np.random.default_rng(2).integers(300, 4000, size=12).tolist())
    step = _Step(case, "int8")
    ref = step.run(None)
    other_cl = step.cl.clone()  # same lengths, another buffer
    _same(step.run(step.plan(cl=other_cl)), ref, "plan of another lengths buffer")
    other_bt = step.bt.clone()
    _same(step.run(step.plan(bt=other_bt)), ref, "plan of another block table")
    _same(step.run(step.plan(max_context_len=step.max_ctx + 1)), ref, "plan of another max_context_len")
    _same(step.run(step.plan(fused=False)), ref, "plan of the unfused kernel")
    junk = torch.full_like(step.plan(), -7)
    _same(step.run(junk), ref, "garbage plan")


def test_plan_of_lengths_rewritten_in_place_is_ignored():
    """A plan records a checksum of the lengths it was made from.  After the
    lengths buffer is rewritten in place (same buffer, same geometry, as a
    serving loop's static buffers are), a launch given the old plan locates
    its work itself, including the first tiles the plan named."""
    rng = np.random.default_rng(21)
    case = make_case(4646, 12, 32, 8, 128, 256, rng.integers(2000, 4000, size=12).tolist())
    step = _Step(case, "int8")
    stale = step.plan()
    new_lens = (case.lens // 3 + rng.integers(1, 200, size=12)).astype(np.int32)
    step.cl.copy_(_t(new_lens))
    fresh = step.plan()
    assert not torch.equal(fresh, stale), "the rewrite must change the plan"
    _same(step.run(stale), step.run(None), "plan of lengths rewritten in place")
    _same(step.run(fresh), step.run(None), "plan of the new lengths")


def test_plan_entries_tile_the_stream():
    """The entries cut the token stream into consecutive slices, and each
    wave's first-tile row is the block-table row of its first tile."""
    bs, hkv = 256, 8
    lens = np.random.default_rng(8).integers(1, 6000, size=40)
    case = make_case(4343, len(lens), 32, hkv, 128, bs, lens)
    step = _Step(case, "int8")
    plan = _np(step.plan()).astype(np.int64)
    hdr = plan[:HEADER]
    assert hdr[0] == 0x50384B53 and hdr[1] == len(lens) and hdr[2] == step.max_ctx and hdr[8] == hkv
    w, ghost = int(hdr[3]), int(hdr[6])
    ent = plan[HEADER: HEADER + ENTRY * w].reshape(w, ENTRY)
    stream = np.where(lens > 0, (lens + 31) // 32 * 32 + ghost, 0)
    total = int(stream.sum())
    starts = np.concatenate([[0], np.cumsum(stream)])
    assert (ent[:, 0] == total).all()
    cut = ent[:, 1] < total  # slices inside the stream (the rest hold nothing)
    lo, hi = ent[cut, 1], ent[cut, 2]
    n_in = int(cut.sum())
    assert cut[:n_in].all() and not cut[n_in:].any(), "the slices inside the stream come first"
    assert lo[0] == 0 and hi[-1] == total and (lo[1:] == hi[:-1]).all() and (lo < hi).all()
    for e in ent[ent[:, 5] > 0]:
        b, pb, L = int(e[3]), int(e[4]), int(e[5])
        assert pb == starts[b] and L == lens[b], "first segment: row start and length"
        s0 = max(int(e[1]), pb + ghost) - (pb + ghost)
        s1 = min(int(e[2]), pb + ghost + (L + 31) // 32 * 32) - (pb + ghost)
        for wv in range(4):
            tb = s0 + 32 * wv
            if tb < min(s1, s0 + 2048, L):
                blk = int(case.block_table[b, tb // bs])
                assert e[12 + wv] == (blk * hkv) * bs + tb % bs, f"row {b}: wave {wv}'s first tile"
            else:
                assert e[12 + wv] == -1


def test_planned_step_graph_replays():
    """The plan launch and three layers' planned decode launches captured in
    one graph: every replay returns the eager outputs and cache bytes."""
    case = make_case(4444, 16, 32, 8, 128, 256, np.random.default_rng(9).integers(200, 5000, size=16).tolist(),
                     outlier_channels=2)
    step = _Step(case, "int8")
    eager = step.run(None)
    caches = [[_t(x) for x in step.pre] for _ in range(3)]
    c = case

    def body():
        plan = ops.attn_paged_decode_plan(caches[0][0], step.bt, step.cl, c.block_size, num_q_heads=c.num_q_heads,
                                          max_context_len=step.max_ctx)
        return [ops.attn_paged_decode_append(step.q, step.kn, step.vn, *cache, step.bt, step.cl, c.block_size,
                                             max_context_len=step.max_ctx, scale=c.scale, plan=plan)
                for cache in caches]

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = body()
    for _ in range(3):
        torch.zeros(1 << 20, device=DEV).add_(1.0)  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        for out, cache in zip(outs, caches):
            _same((_np(out.float()), [_np(x) for x in cache]), eager, "graph replay")


@pytest.mark.parametrize("v_quant", ["int8", "lloydmax3"])
def test_host_cache_decode_step_with_plan(v_quant):
    """PagedKVCache: one plan per step shared by every layer's
    decode_step_static equals the unplanned calls, cache bytes and outputs."""
    import math

    from superl8_serve_amd.paged_cache import PagedKVCache

    hq, hkv, d, bs, layers = 32, 8, 128, 256, 3
    lens = [700, 1, 2500, 256, 90]
    g = torch.Generator(device=DEV).manual_seed(12)
    caches = [PagedKVCache(layers, len(lens), hkv, 4096, d, device=DEV, block_size=bs, v_quant=v_quant)
              for _ in range(2)]
    for c in caches:
        slots = [c.alloc() for _ in lens]
        c.ensure_capacity(slots, [n + 1 for n in lens])
    for layer in range(layers):
        for s, n in zip(slots, lens):
            k = torch.randn(1, hkv, n, d, generator=g, device=DEV).half()
            v = torch.randn(1, hkv, n, d, generator=g, device=DEV).half()
            for c in caches:
                c.write_prefill(layer, k, v, slot=s)
    kn = [torch.randn(len(lens), hkv, d, generator=g, device=DEV).half() for _ in range(layers)]
    vn = [torch.randn(len(lens), hkv, d, generator=g, device=DEV).half() for _ in range(layers)]
    q = [torch.randn(len(lens), hq, 1, d, generator=g, device=DEV).half() for _ in range(layers)]
    bt = caches[0].block_table(slots)
    ctx = [n + 1 for n in lens]
    cl = torch.tensor(ctx, dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(d)
    plan = caches[1].decode_step_plan(bt, cl, max(ctx), num_q_heads=hq)
    for layer in range(layers):
        ref = caches[0].decode_step_static(layer, q[layer], kn[layer], vn[layer], bt, cl, max(ctx), scale=scale)
        out = caches[1].decode_step_static(layer, q[layer], kn[layer], vn[layer], bt, cl, max(ctx), scale=scale,
                                           plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"layer {layer}"
    names = (("k_cache", "k_scale", "v_cache", "v_scale") if v_quant == "int8"
             else ("k_cache", "k_scale", "v_packed", "v_norm"))
    for name in names:
        assert torch.equal(getattr(caches[0], name), getattr(caches[1], name)), name


# ---- adaptive plans (attn_paged_decode_plan(adaptive=True)) ----
AD_MAGIC, AD_BOUNDS = 0x41445053, 8  # adaptive area: magic, W, Hkv, batch, epoch, total, -, -, bounds[W + 1]


def _adaptive_area(plan, hkv):
    """(words of the adaptive area, its bounds, the feedback [hkv, w, 3]:
    epoch, start, end) of a plan tensor."""
    p = _np(plan).astype(np.int64)
    w = int(p[3])
    # header, wmax entries, the adaptive words and wmax + 1 bounds, 3 feedback words per (head, column)
    wmax = (len(p) - HEADER - AD_BOUNDS - 1) // (ENTRY + 1 + 3 * hkv)
    assert HEADER + ENTRY * wmax + AD_BOUNDS + wmax + 1 + 3 * hkv * wmax == len(p)
    ad = p[HEADER + ENTRY * wmax:]
    fb = ad[AD_BOUNDS + wmax + 1:].reshape(hkv, wmax, 3)[:, :w]
    return ad, ad[AD_BOUNDS: AD_BOUNDS + w + 1], fb


def _check_close(a, b, what):
    """Same cache bytes; outputs within the attention tolerance."""
    from tests.kvgpu import assert_close

    out_a, cache_a = a
    out_b, cache_b = b
    for x, y, name in zip(cache_a, cache_b, ("k_cache", "k_scale", "v", "v_scale")):
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), f"{what}: {name} differs"
    assert_close(out_a, out_b, what)


def _qwen_like_case(seed, batch, layout="int8"):
    lens = np.random.default_rng(seed).integers(1500, 5000, size=batch).tolist()
    return _Step(make_case(seed, batch, 32, 8, 128, 256, lens, outlier_channels=2), layout)


@pytest.mark.parametrize("layout", ["int8", "k8v3"])
def test_adaptive_plan_steps(layout):
    """Steps with one adaptive plan tensor: the first plan (zeroed buffer) is
    the fixed split, bit for bit; later ones move the bounds (multiples of 32,
    from 0 to the stream total) and keep the cache bytes, with outputs within
    the attention tolerance of the fixed split's."""
    step = _qwen_like_case(5150, 24, layout)
    ref = step.run(None)
    fixed = _np(step.plan()).astype(np.int64)
    plan = step.plan(adaptive=True)
    ad, bd, _ = _adaptive_area(plan, 8)
    w = int(fixed[3])
    ent = fixed[HEADER: HEADER + ENTRY * w].reshape(w, ENTRY)
    total = int(ent[0, 0])
    assert ad[0] == AD_MAGIC and ad[4] == 1 and ad[5] == total
    assert (np.minimum(ent[:, 1], total) == bd[:w]).all() and bd[w] == total, "first adaptive plan: the fixed split"
    _same(step.run(plan), ref, f"{layout} first adaptive step")
    moved = False
    for k in range(2, 8):
        fb = _adaptive_area(plan, 8)[2]
        assert (fb[:, :, 0] == k - 1).all(), "every workgroup of the last launch recorded its times"
        step.plan(adaptive=True, plan=plan)
        ad, bd, _ = _adaptive_area(plan, 8)
        assert ad[4] == k, "epoch"
        assert bd[0] == 0 and bd[w] == total and (np.diff(bd) >= 0).all() and (bd % 32 == 0).all()
        inner = bd[:w] < total  # slices that start inside the stream hold at least a tile
        assert (np.diff(bd)[inner] >= 32).all()
        moved = moved or not (np.minimum(ent[:, 1], total) == bd[:w]).all()
        _check_close(step.run(plan), ref, f"{layout} adaptive step {k}")
    assert moved, f"the bounds never left the fixed split (adaptive words {ad[:8].tolist()})"


@pytest.mark.parametrize("lens_range", [(1500, 5000), (260, 480)])
def test_adaptive_plan_random_feedback(lens_range):
    """Feedback times planted in the plan buffer (random per workgroup, under
    the plan's epoch) steer the next bounds to skewed splits -- with short
    rows, streams close to the least length that adapts, where shares sit at
    their floor: the bounds stay a partition of the stream (multiples of 32,
    every slice inside the stream at least a tile), cache bytes equal the
    fixed split's and outputs stay within the attention tolerance."""
    rng = np.random.default_rng(77 + lens_range[0])
    lens = rng.integers(lens_range[0], lens_range[1], size=24).tolist()
    step = _Step(make_case(5454 + lens_range[0], 24, 32, 8, 128, 256, lens, outlier_channels=2), "int8")
    ref = step.run(None)
    plan = step.plan(adaptive=True)
    p = _np(plan).astype(np.int64)
    w = int(p[3])
    wmax = (len(p) - HEADER - AD_BOUNDS - 1) // (ENTRY + 1 + 3 * 8)
    fb0 = HEADER + ENTRY * wmax + AD_BOUNDS + wmax + 1
    adapted = 0
    for trial in range(5):
        host = _np(plan).copy()
        ad, bd, _ = _adaptive_area(plan, 8)
        epoch = int(ad[4])
        fb = host[fb0: fb0 + 3 * 8 * wmax].reshape(8, wmax, 3)
        fb[:, :w, 0] = epoch
        fb[:, :w, 1] = 1000
        fb[:, :w, 2] = 1000 + rng.integers(100, 100000, size=(8, w))
        plan.copy_(_t(host))
        step.plan(adaptive=True, plan=plan)
        ad, bd, _ = _adaptive_area(plan, 8)
        total = int(ad[5])
        assert ad[4] == epoch + 1
        assert bd[0] == 0 and bd[w] == total and (np.diff(bd) >= 0).all() and (bd % 32 == 0).all()
        inner = bd[:w] < total
        assert (np.diff(bd)[inner] >= 32).all(), f"trial {trial}: an empty slice inside the stream"
        fixed = _np(step.plan()).astype(np.int64)[HEADER: HEADER + ENTRY * w].reshape(w, ENTRY)
        adapted += int(not (np.minimum(fixed[:, 1], total) == bd[:w]).all())
        _check_close(step.run(plan), ref, f"random feedback trial {trial}")
    assert adapted > 0, "no trial left the fixed split"


def test_adaptive_plan_falls_back_on_new_lengths():
    """After the lengths are rewritten in place (the stream total moves by
    more than a sixteenth), the next adaptive plan is the fixed split again:
    bit-identical outputs to the unplanned launch on the new lengths."""
    rng = np.random.default_rng(31)
    step = _qwen_like_case(5252, 24)
    plan = step.plan(adaptive=True)
    for _ in range(4):
        step.run(plan)
        step.plan(adaptive=True, plan=plan)
    new_lens = (step.case.lens // 2 + rng.integers(1, 200, size=24)).astype(np.int32)
    step.cl.copy_(_t(new_lens))
    step.plan(adaptive=True, plan=plan)
    _same(step.run(plan), step.run(None), "adaptive plan after a length rewrite")


def test_adaptive_plan_graph_replays():
    """The adaptive plan launch and three layers' planned decode launches in
    one graph, replayed: the bounds adapt from replay to replay, every replay
    keeps the cache bytes and stays within tolerance of the eager outputs."""
    step = _qwen_like_case(5353, 24)
    eager = step.run(None)
    caches = [[_t(x) for x in step.pre] for _ in range(3)]
    c = step.case
    plan = step.plan(adaptive=True)

    def body():
        ops.attn_paged_decode_plan(caches[0][0], step.bt, step.cl, c.block_size, num_q_heads=c.num_q_heads,
                                   max_context_len=step.max_ctx, adaptive=True, plan=plan)
        return [ops.attn_paged_decode_append(step.q, step.kn, step.vn, *cache, step.bt, step.cl, c.block_size,
                                             max_context_len=step.max_ctx, scale=c.scale, plan=plan)
                for cache in caches]

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        body()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = body()
    epochs = []
    for _ in range(4):
        torch.zeros(1 << 20, device=DEV).add_(1.0)  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        epochs.append(int(_adaptive_area(plan, 8)[0][4]))
        for out, cache in zip(outs, caches):
            _check_close((_np(out.float()), [_np(x) for x in cache]), eager, "adaptive graph replay")
    assert epochs == list(range(epochs[0], epochs[0] + 4))


def test_plan_smaller_than_the_geometry_needs_is_rejected():
    """A plan buffer shorter than s8kv_decode_plan_size(num_kv_heads) is an
    invalid argument (checked on the host before any launch)."""
    case = make_case(4545, 4, 32, 8, 128, 256, [300, 40, 1000, 7])
    step = _Step(case, "int8")
    plan = step.plan()
    with pytest.raises(ValueError, match="plan"):
        step.run(plan[:HEADER + ENTRY])
    _same(step.run(plan), step.run(None), "full-size plan")
