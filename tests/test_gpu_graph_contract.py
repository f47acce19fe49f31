"""GPU tests of the reference's graph-capture contract, through the C ABI:

* graph-captured prefill (the reference's ``GraphedPrefill``,
  cuda_graph.py:1535-1587): ``enable_graph_prefill`` + ``bind_graph_write_prefill``
  on a scratch slot, ``write_prefill`` captured once, then replayed after
  rebinding to real slots of other lengths -- every replay writes the bytes
  an eager ``write_prefill`` of the real prompt writes, and the padding past
  a shorter prompt writes nothing; with explicit positions (the chunked form)
  too;
* padded decode batches (the reference's ``GraphedDecode``,
  cuda_graph.py:593-637): pad rows point at one scratch slot with position 0
  and ``context_len`` 1.  The real rows' cache bytes equal the unpadded call's
  bit for bit and their outputs are within tolerance of the oracle and of the
  unpadded call (the stream-K split points move with the extra rows, so the
  summation order of a split row may change); pad rows return their own
  token's V.
Each graph is replayed several times with eager work and synchronizations in
between, and every replay is checked."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd.paged_cache import PagedKVCache

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _np(t):
    return t.detach().cpu().numpy()


def _same(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def _slot_rows(cache, slot, n):
    """Storage rows [n * Hkv] of positions 0..n-1 of `slot` (one layer)."""
    sm = np.asarray(cache.flat_slot_mapping(slot, n))
    return O.flat_rows(sm, cache.num_kv_heads, cache.block_size).reshape(-1)


def _layer(cache):
    return [_np(t[0]).reshape(cache.num_blocks * cache.num_kv_heads * cache.block_size, -1) for t in cache._tensors()]


@pytest.mark.parametrize("v_quant", ["int8", "lloydmax3"])
def test_graph_captured_prefill_rebinds_to_real_slots(v_quant):
    hkv, d, bs, bucket = 4, 128, 16, 64
    gen = torch.Generator(device=DEV).manual_seed(11)
    cache = PagedKVCache(1, 6, hkv, 256, d, device=DEV, block_size=bs, v_quant=v_quant)
    eager = PagedKVCache(1, 6, hkv, 256, d, device=DEV, block_size=bs, v_quant=v_quant)
    scratch = cache.alloc()
    assert eager.alloc() == scratch
    cache.ensure_capacity([scratch], [bucket])
    eager.ensure_capacity([scratch], [bucket])
    k_static = torch.zeros((1, hkv, bucket, d), dtype=torch.float16, device=DEV)
    v_static = torch.zeros_like(k_static)
    eager.write_prefill(0, k_static, v_static, slot=scratch)  # what the warm-up and capture write
    cache.enable_graph_prefill(bucket)
    cache.bind_graph_write_prefill(scratch, bucket)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        cache.write_prefill(0, k_static, v_static, slot=scratch)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cache.write_prefill(0, k_static, v_static, slot=scratch)
    for n in (50, 17, 64, 33):
        slot = cache.alloc()
        assert eager.alloc() == slot
        cache.ensure_capacity([slot], [n])
        eager.ensure_capacity([slot], [n])
        k = torch.randn((1, hkv, bucket, d), generator=gen, device=DEV).half()
        v = torch.randn((1, hkv, bucket, d), generator=gen, device=DEV).half()
        k_static.copy_(k)
        v_static.copy_(v)
        cache.bind_graph_write_prefill(slot, n)
        g.replay()
        # eager work between replays: the same prompt written the reference's way
        eager.write_prefill(0, k[:, :, :n], v[:, :, :n], slot=slot)
        torch.cuda.synchronize()
        got, want = _layer(cache), _layer(eager)
        rows = _slot_rows(cache, slot, n)
        for a, b in zip(got, want):
            assert _same(a[rows], b[rows]), f"replay for a {n}-token prompt differs from the eager write"
        # padding tokens write nothing: every row outside the real prompt is
        # what the eager twin holds (the capture-time writes of the scratch
        # slot, then nothing else)
        keep = np.ones(got[0].shape[0], bool)
        keep[rows] = False
        for a, b in zip(got, want):
            assert _same(a[keep], b[keep]), "a padding token was written outside the real prompt"
        cache.free(slot)
        eager.free(slot)


def test_graph_captured_chunk_prefill_with_positions():
    """The chunked form: ``write_prefill(..., positions=)`` captured against
    the static block table (kv_cache.py:1047-1058), replayed for other slots."""
    hkv, d, bs, chunk = 4, 64, 16, 48
    gen = torch.Generator(device=DEV).manual_seed(12)
    cache = PagedKVCache(1, 5, hkv, 256, d, device=DEV, block_size=bs)
    eager = PagedKVCache(1, 5, hkv, 256, d, device=DEV, block_size=bs)
    scratch = cache.alloc()
    eager.alloc()
    cache.ensure_capacity([scratch], [200])
    eager.ensure_capacity([scratch], [200])
    k_static = torch.zeros((1, hkv, chunk, d), dtype=torch.float16, device=DEV)
    v_static = torch.zeros_like(k_static)
    pos_static = torch.arange(100, 100 + chunk, device=DEV)
    cache.enable_graph_prefill(256)
    cache.bind_graph_write_prefill(scratch, 200)
    cache.write_prefill(0, k_static, v_static, slot=scratch, positions=pos_static)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        cache.write_prefill(0, k_static, v_static, slot=scratch, positions=pos_static)
    for start in (0, 37, 150):
        slot = cache.alloc()
        assert eager.alloc() == slot
        cache.ensure_capacity([slot], [start + chunk])
        eager.ensure_capacity([slot], [start + chunk])
        k = torch.randn((1, hkv, chunk, d), generator=gen, device=DEV).half()
        v = torch.randn((1, hkv, chunk, d), generator=gen, device=DEV).half()
        pos = torch.arange(start, start + chunk, device=DEV)
        k_static.copy_(k)
        v_static.copy_(v)
        pos_static.copy_(pos)
        cache.bind_graph_write_prefill(slot, start + chunk)
        g.replay()
        eager.write_prefill(0, k, v, slot=slot, positions=pos)
        torch.cuda.synchronize()
        sm = np.asarray(cache.flat_slot_mapping(slot, start + chunk))[start:]
        rows = O.flat_rows(sm, hkv, bs).reshape(-1)
        for a, b in zip(_layer(cache), _layer(eager)):
            assert _same(a[rows], b[rows]), f"chunk replay at start {start} differs from the eager write"
        cache.free(slot)
        eager.free(slot)


@pytest.mark.parametrize("fused", [False, True], ids=["decode", "decode_append"])
def test_graph_decode_pad_rows_at_one_scratch_slot(fused):
    """B real rows + pad rows (scratch slot, position 0, context_len 1),
    captured once, replayed over three steps with new tokens."""
    hq, hkv, d, bs = 16, 4, 128, 16
    real, bucket = 5, 12
    rng = np.random.default_rng(13)
    gen = torch.Generator(device=DEV).manual_seed(13)
    scale = 1.0 / math.sqrt(d)
    cache = PagedKVCache(1, 8, hkv, 512, d, device=DEV, block_size=bs)
    plain = PagedKVCache(1, 8, hkv, 512, d, device=DEV, block_size=bs)
    scratch = cache.alloc()
    plain.alloc()
    cache.ensure_capacity([scratch], [1])
    plain.ensure_capacity([scratch], [1])
    slots = [cache.alloc() for _ in range(real)]
    assert [plain.alloc() for _ in range(real)] == slots
    lens = [int(x) for x in rng.integers(30, 400, size=real)]
    for s, n in zip(slots, lens):
        cache.ensure_capacity([s], [n + 3])
        plain.ensure_capacity([s], [n + 3])
        k = torch.randn((1, hkv, n, d), generator=gen, device=DEV).half()
        v = torch.randn((1, hkv, n, d), generator=gen, device=DEV).half()
        cache.write_prefill(0, k, v, slot=s)
        plain.write_prefill(0, k, v, slot=s)
    # graph inputs of the padded bucket
    width = cache.max_blocks_per_seq
    q_st = torch.zeros((bucket, hq, 1, d), dtype=torch.float16, device=DEV)
    k_st = torch.zeros((bucket, hkv, d), dtype=torch.float16, device=DEV)
    v_st = torch.zeros_like(k_st)
    bt_st = torch.zeros((bucket, width), dtype=torch.int32, device=DEV)
    cl_st = torch.ones(bucket, dtype=torch.int32, device=DEV)
    sm_st = torch.zeros(bucket, dtype=torch.int32, device=DEV)
    max_ctx = 512

    def fill(step):
        b_slots = slots + [scratch] * (bucket - real)
        positions = [n + step for n in lens] + [0] * (bucket - real)
        cache.fill_block_table(bt_st, b_slots)
        cache.fill_slot_mapping(sm_st, b_slots, positions)
        cl_st.copy_(torch.tensor([p + 1 for p in positions], dtype=torch.int32))
        return positions

    def layer_step():
        if fused:
            return cache.decode_step_static(0, q_st, k_st, v_st, bt_st, cl_st, max_ctx, scale=scale)
        cache.write_decode_static(0, sm_st, k_st, v_st)
        return cache.decode_attn_static(0, q_st, bt_st, cl_st, max_ctx, scale=scale)

    fill(0)
    layer_step()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out_st = layer_step()
    for step in range(3):
        positions = fill(step)
        q = torch.randn((bucket, hq, 1, d), generator=gen, device=DEV).half()
        kn = torch.randn((bucket, hkv, d), generator=gen, device=DEV).half()
        vn = torch.randn((bucket, hkv, d), generator=gen, device=DEV).half()
        q_st.copy_(q)
        k_st.copy_(kn)
        v_st.copy_(vn)
        g.replay()
        got = out_st.clone()
        # the same step unpadded, eagerly, on the twin cache
        ctx = [p + 1 for p in positions[:real]]
        if fused:
            want = plain.decode_step(0, q[:real], kn[:real], vn[:real], slots, positions[:real], scale=scale)
        else:
            plain.write_decode(0, slots, positions[:real], kn[:real], vn[:real])
            want = plain.decode_attn(0, q[:real], slots, positions[:real], scale=scale)
        torch.cuda.synchronize()
        rows = np.concatenate([_slot_rows(cache, s, c) for s, c in zip(slots, ctx)])
        for a, b in zip(_layer(cache), _layer(plain)):
            assert _same(a[rows], b[rows]), f"step {step}: a real row's cache bytes differ from the unpadded call"
        layer = O.LayerCache(*[_np(t[0]) for t in cache._tensors()])
        bt = _np(cache.block_table(slots))
        ref = O.paged_decode(_np(q[:real])[:, :, 0, :], layer, bt, np.asarray(ctx), scale)
        g_np = _np(got.float())[:real, :, 0, :]
        mx, rel = O.attention_errors(g_np, ref)
        assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"step {step}: real rows {mx:.3e} / {rel:.3e}"
        mx, rel = O.attention_errors(g_np, _np(want.float())[:, :, 0, :].astype(np.float64))
        assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"step {step}: padded vs unpadded {mx:.3e}"
        if fused:  # a pad row attends only its own new token: its V, exactly dequantized
            vq, vs = O.quantize_i8_rowwise(_np(vn[real:]))
            own = (vq.astype(np.float64) * vs[..., None])  # [pads, Hkv, D]
            want_pad = np.repeat(own, hq // hkv, axis=1)
            mx, rel = O.attention_errors(_np(got.float())[real:, :, 0, :], want_pad)
            assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"step {step}: pad rows {mx:.3e}"
