"""GPU parity of the one-launch decode step (``attn_paged_decode_append``:
append row b's new token at position context_lens[b]-1, then attend) against
the separate append + decode ops and against the oracle, through the C ABI.

The fused op must leave the cache byte-identical to the oracle's append and
return exactly what ``quantize_kv_write_paged`` followed by
``attn_paged_decode_cached`` returns (same slicing, same arithmetic)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import empty_int8_cache, empty_k8v3_cache, make_case

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _np(t):
    return t.detach().cpu().numpy()


def _split(case):
    """Oracle cache holding every token but each row's last, the full oracle
    cache, the rows' last tokens [B, Hkv, D] and their slots (-1: empty row)."""
    ends = np.cumsum(case.lens)
    last = ends - 1
    has = case.lens > 0
    keep = np.ones(int(ends[-1]) if len(ends) else 0, bool)
    keep[last[has]] = False
    pre = empty_int8_cache(case)
    O.quantize_kv_write_paged(case.k[keep], case.v[keep], *pre, case.slots[keep])
    full = empty_int8_cache(case)
    O.quantize_kv_write_paged(case.k, case.v, *full, case.slots)
    k_new = np.zeros((case.batch, case.num_kv_heads, case.head_dim), np.float16)
    v_new = np.zeros_like(k_new)
    k_new[has] = case.k[last[has]]
    v_new[has] = case.v[last[has]]
    slots = np.where(has, case.slots[np.minimum(last, len(case.slots) - 1)] if len(case.slots) else -1, -1)
    return pre, full, k_new, v_new, slots.astype(np.int32)


def _fused(case, pre, k_new, v_new, lens, max_ctx):
    kc, ks, vc, vs = (_t(x) for x in pre)
    q = _t(case.q)[:, :, None, :]
    out = ops.attn_paged_decode_append(q, _t(k_new), _t(v_new), kc, ks, vc, vs, _t(case.block_table),
                                       _t(np.asarray(lens, np.int32)), case.block_size, max_context_len=max_ctx,
                                       scale=case.scale)
    torch.cuda.synchronize()
    return _np(out.float())[:, :, 0, :], [_np(x) for x in (kc, ks, vc, vs)]


def _separate(case, pre, k_new, v_new, slots, lens, max_ctx):
    kc, ks, vc, vs = (_t(x) for x in pre)
    ops.quantize_kv_write_paged(_t(k_new), _t(v_new), kc, ks, vc, vs, _t(slots))
    q = _t(case.q)[:, :, None, :]
    out = ops.attn_paged_decode_cached(q, kc, ks, vc, vs, _t(case.block_table), _t(np.asarray(lens, np.int32)),
                                       case.block_size, max_context_len=max_ctx, scale=case.scale)
    torch.cuda.synchronize()
    return _np(out.float())[:, :, 0, :], [_np(x) for x in (kc, ks, vc, vs)]


def _check(case, max_ctx=None, what="fused"):
    max_ctx = int(case.lens.max()) if max_ctx is None else max_ctx
    pre, full, k_new, v_new, slots = _split(case)
    got, cache = _fused(case, pre, k_new, v_new, case.lens, max_ctx)
    for a, b, name in zip(cache, full, ("k_cache", "k_scale", "v_cache", "v_scale")):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{what}: {name} differs from the oracle's append"
    ref = O.paged_decode(case.q, O.LayerCache(*full), case.block_table, case.lens, case.scale)
    mx, rel = O.attention_errors(got, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"
    sep, _ = _separate(case, pre, k_new, v_new, slots, case.lens, max_ctx)
    assert np.array_equal(got, sep), f"{what}: differs from append + decode (max {np.abs(got - sep).max():.3e})"


@pytest.mark.parametrize("hq,hkv,d,bs,lens", [
    (32, 8, 128, 256, "qwen"),                       # Qwen3-8B heads, ragged lengths
    (16, 8, 128, 16, [100, 17, 16, 15, 1, 0]),       # first token (L=1), empty row, block edges
    (16, 8, 128, 256, [256, 257, 512, 255]),         # new token first / last in its block
    (8, 2, 256, 16, [50, 129]),
    (8, 4, 64, 8, [33, 2, 80]),
    (4, 2, 32, 4, [9, 31, 12, 1]),                   # tiles cross blocks
    (16, 1, 128, 32, [70]),                          # 16 q heads on one kv head
])
def test_decode_append_matches_append_then_decode(hq, hkv, d, bs, lens):
    if lens == "qwen":
        lens = np.random.default_rng(3).integers(200, 3000, size=16).tolist()
    case = make_case(2000 + hq + d + bs, len(lens), hq, hkv, d, bs, lens, outlier_channels=2 if d == 128 else 0)
    _check(case)


@pytest.mark.parametrize("wg_per_head,ghost,batch,bs,lens", [
    (1, 128, 4, 16, [1000, 129, 5000, 0]),           # one slice per head, rows past 2048 tokens
    (2, 0, 4, 256, [5000, 100, 0, 37]),              # the last tile in a later block-id stage of a split row
    (7, 0, 64, 32, "short"),                         # rows split across slices
    (40, 512, 64, 16, "short"),                      # slices holding no tokens
    (3, 64, 5, 8, [300, 1, 64, 2500, 31]),           # block_size < 32
])
def test_decode_append_slicings(wg_per_head, ghost, batch, bs, lens, monkeypatch):
    """The appending workgroup is the one holding the row's last tile, wherever
    the slicing puts it."""
    monkeypatch.setenv("S8KV_DECODE_WG_PER_HEAD", str(wg_per_head))
    monkeypatch.setenv("S8KV_DECODE_GHOST", str(ghost))
    if lens == "short":
        lens = np.random.default_rng(6).integers(0, 120, size=batch).tolist()
    case = make_case(77 + wg_per_head, batch, 32, 8, 128, bs, lens)
    _check(case, what=f"fused wg/head={wg_per_head}")


def test_decode_append_rows_past_max_context_len():
    """A row longer than max_context_len attends its first max_context_len
    tokens and appends nothing (as the separate ops do with a skipped slot)."""
    case = make_case(91, 3, 16, 8, 128, 16, [300, 500, 40], width=32)
    pre, full, k_new, v_new, slots = _split(case)
    slots[1] = -1  # the separate path skips the truncated row's append too
    got, cache = _fused(case, pre, k_new, v_new, case.lens, 400)
    sep, sep_cache = _separate(case, pre, k_new, v_new, slots, case.lens, 400)
    for a, b in zip(cache, sep_cache):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    assert np.array_equal(got, sep)


def test_decode_append_graph_replays():
    """Captured in a HIP graph: every replay (the append rewrites the same
    bytes) returns the eager result and leaves the same cache."""
    case = make_case(93, 8, 32, 8, 128, 256, [700, 1, 256, 3000, 90, 1500, 257, 33])
    pre, full, k_new, v_new, _ = _split(case)
    eager, _ = _fused(case, pre, k_new, v_new, case.lens, int(case.lens.max()))
    kc, ks, vc, vs = (_t(x) for x in pre)
    q = _t(case.q)[:, :, None, :]
    kn, vn, bt, cl = _t(k_new), _t(v_new), _t(case.block_table), _t(case.lens.astype(np.int32))
    mc = int(case.lens.max())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.attn_paged_decode_append(q, kn, vn, kc, ks, vc, vs, bt, cl, case.block_size, max_context_len=mc,
                                     scale=case.scale)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = ops.attn_paged_decode_append(q, kn, vn, kc, ks, vc, vs, bt, cl, case.block_size, max_context_len=mc,
                                           scale=case.scale)
    for _ in range(3):
        torch.zeros(1 << 20, device=DEV).add_(1.0)  # eager work between replays
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(_np(out.float())[:, :, 0, :], eager)
    for a, b in zip((kc, ks, vc, vs), full):
        assert np.array_equal(_np(a).view(np.uint8), b.view(np.uint8))


# ---------------------------------------------------------------------------
# K8V3 layout (int8 K, 3-bit Lloyd-Max V)
# ---------------------------------------------------------------------------

CODEBOOK = O.gaussian_codebook(3, 128)


def _split_k8v3(case):
    ends = np.cumsum(case.lens)
    last = ends - 1
    has = case.lens > 0
    keep = np.ones(int(ends[-1]) if len(ends) else 0, bool)
    keep[last[has]] = False
    pre = empty_k8v3_cache(case)
    O.k8v3_write_paged(case.k[keep], case.v[keep], *pre, CODEBOOK, case.slots[keep])
    full = empty_k8v3_cache(case)
    O.k8v3_write_paged(case.k, case.v, *full, CODEBOOK, case.slots)
    k_new = np.zeros((case.batch, case.num_kv_heads, case.head_dim), np.float16)
    v_new = np.zeros_like(k_new)
    k_new[has] = case.k[last[has]]
    v_new[has] = case.v[last[has]]
    slots = np.where(has, case.slots[np.minimum(last, len(case.slots) - 1)], -1).astype(np.int32)
    return pre, full, k_new, v_new, slots


@pytest.mark.parametrize("hq,hkv,d,bs,lens", [
    (32, 8, 128, 256, "long"),                       # Qwen3-8B heads, 8k-32k-like rows (shortened)
    (16, 8, 128, 16, [100, 17, 16, 15, 1, 0]),
    (8, 2, 256, 16, [50, 129, 300]),                 # two Lloyd-Max blocks per row
])
def test_decode_append_k8v3_matches_append_then_decode(hq, hkv, d, bs, lens):
    if lens == "long":
        lens = np.random.default_rng(4).integers(1500, 6000, size=8).tolist()
    case = make_case(3000 + hq + d + bs, len(lens), hq, hkv, d, bs, lens, outlier_channels=2 if d == 128 else 0)
    max_ctx = int(case.lens.max())
    pre, full, k_new, v_new, slots = _split_k8v3(case)
    cb = _t(CODEBOOK)
    q = _t(case.q)[:, :, None, :]
    bt, cl = _t(case.block_table), _t(case.lens.astype(np.int32))
    kc, ks, vp, vn = (_t(x) for x in pre)
    got = ops.attn_paged_decode_append_k8v3(q, _t(k_new), _t(v_new), kc, ks, vp, vn, cb, bt, cl, case.block_size,
                                            max_context_len=max_ctx, scale=case.scale)
    torch.cuda.synchronize()
    for a, b, name in zip((kc, ks, vp, vn), full, ("k_cache", "k_scale", "v_packed", "v_norm")):
        assert np.array_equal(_np(a).view(np.uint8), b.view(np.uint8)), f"{name} differs from the oracle's append"
    got = _np(got.float())[:, :, 0, :]
    layer = O.LayerCache(*full[:2], v_packed=full[2], v_norm=full[3], v_codebook=CODEBOOK)
    ref = O.paged_decode(case.q, layer, case.block_table, case.lens, case.scale)
    mx, rel = O.attention_errors(got, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"k8v3 fused: max err {mx:.3e}, rel rms {rel:.3e}"
    kc2, ks2, vp2, vn2 = (_t(x) for x in pre)
    ops.quantize_kv_write_paged_k8v3(_t(k_new), _t(v_new), kc2, ks2, vp2, vn2, cb, _t(slots))
    sep = ops.attn_paged_decode_k8v3(q, kc2, ks2, vp2, vn2, cb, bt, cl, case.block_size, max_context_len=max_ctx,
                                     scale=case.scale)
    torch.cuda.synchronize()
    assert np.array_equal(got, _np(sep.float())[:, :, 0, :]), "k8v3 fused differs from append + decode"
