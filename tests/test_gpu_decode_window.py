"""GPU parity of the sliding-window paged decode (row b attends its last
`window` tokens) against the float64 oracle, through the C ABI.

The reference's sliding-window layers read the window back dense and decode
per row (gqa_attention.py:191-196, kv_cache.py:1233-1299); the oracle restates
that range, [max(0, L - window), L).  Tolerance as for decode:
max(|out-ref| / max(1,|ref|)) <= 2e-3 and relative RMS <= 1e-3.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import make_case, oracle_fill_int8, oracle_fill_k8v3

pytestmark = pytest.mark.gpu

DEV = "cuda"
CODEBOOK = O.gaussian_codebook(3, 128)


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _close(out, ref, what):
    mx, rel = O.attention_errors(out, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"


def _int8(case, cache, window, q=None):
    kc, ks, vc, vs = (_t(x) for x in cache)
    q = _t(case.q if q is None else q)[:, :, None, :]
    args = (q, kc, ks, vc, vs, _t(case.block_table), _t(case.lens.astype(np.int32)), case.block_size)
    kw = dict(max_context_len=int(case.lens.max()), scale=case.scale)
    out = ops.attn_paged_decode_cached(*args, **kw) if window is None else \
        ops.attn_paged_decode_window(*args, window=window, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()[:, :, 0, :]


def _k8v3(case, cache, window):
    kc, ks, vp, vn = (_t(x) for x in cache)
    q = _t(case.q)[:, :, None, :]
    args = (q, kc, ks, vp, vn, _t(CODEBOOK), _t(case.block_table), _t(case.lens.astype(np.int32)), case.block_size)
    kw = dict(max_context_len=int(case.lens.max()), scale=case.scale)
    out = ops.attn_paged_decode_k8v3(*args, **kw) if window is None else \
        ops.attn_paged_decode_window_k8v3(*args, window=window, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()[:, :, 0, :]


@pytest.mark.parametrize("hq,hkv,d,bs,lens,window", [
    (8, 2, 128, 16, [300, 37, 256, 1, 0, 4100], 100),    # window inside, shorter rows, empty row
    (8, 2, 128, 256, [700, 2600, 31, 33], 33),           # start not on a 32-token tile
    (32, 8, 128, 256, [5000, 4096, 4097, 300], 4096),    # window = a row's length, long rows
    (16, 16, 64, 4, [90, 17, 64], 5),                    # tiny blocks (tiles cross blocks), G = 1
    (4, 2, 256, 16, [120, 257], 64),                     # head_dim 256
    (8, 2, 32, 16, [45, 80], 1),                         # window 1: the last token's V
    (64, 4, 128, 16, [2000, 999, 1500], 1000),           # G = 16
])
def test_window_decode_int8(hq, hkv, d, bs, lens, window):
    case = make_case(300 + d + bs + window, len(lens), hq, hkv, d, bs, lens, outlier_channels=2)
    cache = oracle_fill_int8(case)
    ref = O.paged_decode(case.q, O.LayerCache(*cache), case.block_table, case.lens, case.scale, window=window)
    _close(_int8(case, cache, window), ref, f"window {window}")


@pytest.mark.parametrize("d,bs,lens,window", [(128, 16, [300, 4100, 7], 200), (256, 256, [1000, 260], 77)])
def test_window_decode_k8v3(d, bs, lens, window):
    case = make_case(400 + d + window, len(lens), 8, 2, d, bs, lens, outlier_channels=2)
    cache = oracle_fill_k8v3(case, CODEBOOK)
    layer = O.LayerCache(cache[0], cache[1], v_packed=cache[2], v_norm=cache[3], v_codebook=CODEBOOK)
    ref = O.paged_decode(case.q, layer, case.block_table, case.lens, case.scale, window=window)
    _close(_k8v3(case, cache, window), ref, f"k8v3 window {window}")


def test_window_covering_every_row_equals_full_decode():
    """A window at least as long as every row views each row from position 0:
    the same slices and the same arithmetic as the unwindowed decode."""
    case = make_case(451, 5, 8, 2, 128, 16, [300, 37, 256, 1, 900])
    cache = oracle_fill_int8(case)
    assert np.array_equal(_int8(case, cache, 900), _int8(case, cache, None))
    kcase = make_case(452, 3, 8, 2, 128, 16, [300, 37, 900])
    kcache = oracle_fill_k8v3(kcase, CODEBOOK)
    assert np.array_equal(_k8v3(kcase, kcache, 5000), _k8v3(kcase, kcache, None))


def test_tokens_outside_the_window_are_not_read_into_the_result():
    """Garbage K and non-finite scales before the window (in the window's
    first tile and in earlier blocks) leave the windowed output unchanged."""
    case = make_case(461, 3, 8, 2, 128, 16, [300, 150, 77], outlier_channels=1)
    cache = oracle_fill_int8(case)
    window = 45
    before = _int8(case, cache, window)
    kc, ks, vc, vs = (x.copy() for x in cache)
    for b, n in enumerate(case.lens):
        for p in range(max(0, int(n) - window)):
            blk, off = case.block_table[b, p // case.block_size], p % case.block_size
            kc[blk, :, off] = 127
            ks[blk, :, off] = np.inf
            vc[blk, :, off] = -127
            vs[blk, :, off] = np.nan
    after = _int8(case, (kc, ks, vc, vs), window)
    assert np.all(np.isfinite(after))
    assert np.array_equal(after, before)


def test_window_must_be_positive():
    case = make_case(471, 1, 4, 2, 128, 16, [20])
    cache = oracle_fill_int8(case)
    with pytest.raises(ValueError, match="window"):
        _int8(case, cache, 0)


def test_host_cache_windowed_decode():
    """PagedKVCache.decode_attn(window=...) routes to the windowed kernel."""
    from superl8_serve_amd.paged_cache import PagedKVCache

    g = torch.Generator(device=DEV).manual_seed(5)
    hq, hkv, d, bs = 8, 2, 128, 16
    for v_quant in ("int8", "lloydmax3"):
        c = PagedKVCache(1, 2, hkv, 512, d, device=DEV, block_size=bs, v_quant=v_quant)
        slots = [c.alloc(), c.alloc()]
        lens = [200, 61]
        c.ensure_capacity(slots, lens)
        for s, n in zip(slots, lens):
            k = torch.randn(1, hkv, n, d, generator=g, device=DEV).half()
            c.write_prefill(0, k, torch.randn_like(k), slot=s)
        q = torch.randn(2, hq, 1, d, generator=g, device=DEV).half()
        out = c.decode_attn(0, q, slots, [n - 1 for n in lens], scale=0.1, window=50)
        r = c._layer_row(0)
        if v_quant == "lloydmax3":
            layer = O.LayerCache(c.k_cache[r].cpu().numpy(), c.k_scale[r].cpu().numpy(),
                                 v_packed=c.v_packed[r].cpu().numpy(), v_norm=c.v_norm[r].cpu().numpy(),
                                 v_codebook=c.v_codebook[r].cpu().numpy())
        else:
            layer = O.LayerCache(c.k_cache[r].cpu().numpy(), c.k_scale[r].cpu().numpy(), c.v_cache[r].cpu().numpy(),
                                 c.v_scale[r].cpu().numpy())
        ref = O.paged_decode(q[:, :, 0].cpu().numpy(), layer, c.block_table(slots).cpu().numpy(), np.array(lens), 0.1,
                             window=50)
        _close(out[:, :, 0].float().cpu().numpy(), ref, f"{v_quant} via cache")


# ---------------------------------------------------------------------------
# verify attention of a sliding-window layer: the last `window` prefix keys
# plus the drafts (gqa_attention.py:305-314)
# ---------------------------------------------------------------------------


def _verify_case(seed, batch, hq, hkv, d, bs, prefix, nq, k8v3=False):
    prefix = np.asarray(prefix)
    case = make_case(seed, batch, hq, hkv, d, bs, prefix + nq, outlier_channels=2)
    cache = oracle_fill_k8v3(case, CODEBOOK) if k8v3 else oracle_fill_int8(case)
    q = np.random.default_rng(seed + 7).standard_normal((batch, hq, nq, d)).astype(np.float16)
    return case, cache, q, prefix


def _verify(case, cache, q, prefix, window, k8v3=False, tree_mask=None):
    c = [_t(x) for x in cache]
    kw = dict(tree_mask=None if tree_mask is None else _t(tree_mask),
              max_context_len=int(case.block_table.shape[1] * case.block_size), scale=case.scale, window=window)
    bt, pl = _t(case.block_table), _t(prefix.astype(np.int32))
    if k8v3:
        out = ops.attn_paged_verify_k8v3(_t(q), *c, _t(CODEBOOK), bt, pl, case.block_size, **kw)
    else:
        out = ops.attn_paged_verify(_t(q), *c, bt, pl, case.block_size, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _verify_ref(case, cache, q, prefix, window, k8v3=False, tree_mask=None):
    layer = O.LayerCache(cache[0], cache[1], v_packed=cache[2], v_norm=cache[3], v_codebook=CODEBOOK) if k8v3 \
        else O.LayerCache(*cache)
    return O.paged_verify(q, layer, case.block_table, prefix, case.scale, tree_mask=tree_mask, window=window)


@pytest.mark.parametrize("k8v3,hq,hkv,d,bs,prefix,nq,window", [
    (False, 8, 2, 128, 16, [1000, 37, 300], 6, 300),     # chain: one row shorter than the window
    (False, 8, 2, 128, 256, [777, 64], 200, 100),        # a 200-query chunk
    (False, 16, 16, 64, 4, [90, 50], 5, 33),             # tiny blocks, G = 1
    (True, 8, 2, 128, 16, [1000, 130], 9, 129),          # K8V3
    (True, 4, 2, 256, 16, [700, 260], 4, 70),            # K8V3 head_dim 256
])
def test_window_verify(k8v3, hq, hkv, d, bs, prefix, nq, window):
    case, cache, q, pre = _verify_case(600 + d + window, len(prefix), hq, hkv, d, bs, prefix, nq, k8v3)
    _close(_verify(case, cache, q, pre, window, k8v3), _verify_ref(case, cache, q, pre, window, k8v3),
           f"verify window {window}")


def test_window_tree_verify():
    rng = np.random.default_rng(5)
    case, cache, q, pre = _verify_case(611, 2, 16, 4, 128, 16, [2048, 500], 16)
    masks = []
    for _ in range(2):
        m = []
        for i in range(16):
            parent = int(rng.integers(0, i)) if i else -1
            m.append((m[parent] if parent >= 0 else 0) | (1 << i))
        masks.append(m)
    masks = np.array(masks, np.int64)
    _close(_verify(case, cache, q, pre, 400, tree_mask=masks), _verify_ref(case, cache, q, pre, 400, tree_mask=masks),
           "tree verify window")


def test_window_verify_covering_the_prefix_equals_verify():
    """A window covering every row's prefix masks nothing.  Both calls run the
    32-row kernel, but the windowed one plans its key split over the window
    and the drafts, not the whole context, so its partial sums may round
    differently: equal within the attention tolerance (a masking error would
    be far outside it), and both match the oracle."""
    from tests.kvgpu import assert_close

    case, cache, q, pre = _verify_case(621, 3, 8, 2, 128, 16, [300, 37, 256], 7)
    windowed, plain = _verify(case, cache, q, pre, 300), _verify(case, cache, q, pre, None)
    assert_close(windowed, plain, "window covering the prefix vs no window")
    ref = _verify_ref(case, cache, q, pre, None)
    assert_close(windowed, ref, "windowed vs oracle")
    assert_close(plain, ref, "unwindowed vs oracle")


@pytest.mark.parametrize("k8v3", [False, True])
def test_window_verify_ignores_keys_before_the_window(k8v3):
    """Cache rows below the window (its first tile holds some) may hold any
    bytes and scales, inf and NaN included: the result is bit-identical."""
    case, cache, q, pre = _verify_case(631, 2, 8, 2, 128, 16, [400, 150], 5, k8v3)
    window = 61
    before = _verify(case, cache, q, pre, window, k8v3)
    kc, ks, vc, vs = (x.copy() for x in cache)
    for b, p in enumerate(pre):
        for pos in range(max(0, int(p) - window)):
            blk, off = case.block_table[b, pos // case.block_size], pos % case.block_size
            kc[blk, :, off] = 127
            ks[blk, :, off] = np.inf if pos % 2 else np.nan  # non-finite scales must not reach the output
            vc[blk, :, off] = -1 if k8v3 else -127
            vs[blk, :, off] = np.nan if pos % 2 else np.inf
    assert np.array_equal(_verify(case, (kc, ks, vc, vs), q, pre, window, k8v3), before)


def _drafts(case, pre, nq):
    """The fresh fp16 K / V of every row's drafts, [B, S, Hkv, D] (the tokens
    the cache holds quantized at positions prefix .. prefix + S - 1)."""
    starts = np.concatenate([[0], np.cumsum(case.lens)])
    idx = np.stack([starts[b] + pre[b] + np.arange(nq) for b in range(case.batch)])
    return case.k[idx], case.v[idx]


@pytest.mark.parametrize("k8v3,hq,hkv,d,bs,prefix,nq,window", [
    (False, 8, 2, 128, 16, [1000, 37, 300], 6, 300),
    (False, 16, 16, 64, 4, [90, 50], 5, 33),
    (False, 8, 2, 256, 256, [777, 64], 40, 100),
    (True, 8, 2, 128, 16, [1000, 130], 9, 129),
    (True, 4, 2, 256, 16, [700, 260], 4, 70),
    (False, 32, 8, 128, 16, [3000, 500, 45], 40, 1024),  # drafts across tiles, two 128-row blocks
    (True, 32, 8, 128, 256, [2100, 64], 33, 512),
    (False, 64, 4, 128, 32, [2500, 31], 12, 700),        # G = 16, a prefix shorter than a tile
])
def test_window_verify_with_fresh_drafts(k8v3, hq, hkv, d, bs, prefix, nq, window):
    """The reference's window verify attends the prefix window read back from
    the cache plus the drafts' fresh fp16 K / V (gqa_attention.py:298-313):
    against the oracle in that mode, with the drafts passed as a
    [B, Hkv, S, D] -> [B, S, Hkv, D] transpose view; and not the
    cache-roundtripped result."""
    case, cache, q, pre = _verify_case(700 + d + window, len(prefix), hq, hkv, d, bs, prefix, nq, k8v3)
    kd, vd = _drafts(case, pre, nq)
    c = [_t(x) for x in cache]
    kw = dict(max_context_len=int(case.block_table.shape[1] * case.block_size), scale=case.scale, window=window,
              k_draft=_t(kd.transpose(0, 2, 1, 3)).transpose(1, 2), v_draft=_t(vd.transpose(0, 2, 1, 3)).transpose(1, 2))
    bt, pl = _t(case.block_table), _t(pre.astype(np.int32))
    if k8v3:
        out = ops.attn_paged_verify_k8v3(_t(q), *c, _t(CODEBOOK), bt, pl, case.block_size, **kw)
    else:
        out = ops.attn_paged_verify(_t(q), *c, bt, pl, case.block_size, **kw)
    got = out.float().cpu().numpy()
    layer = O.LayerCache(cache[0], cache[1], v_packed=cache[2], v_norm=cache[3], v_codebook=CODEBOOK) if k8v3 \
        else O.LayerCache(*cache)
    ref = O.paged_verify(q, layer, case.block_table, pre, case.scale, window=window, fresh_drafts=(kd, vd))
    _close(got, ref, f"verify window {window} with fresh drafts")
    assert not np.array_equal(got, _verify(case, cache, q, pre, window, k8v3))


@pytest.mark.parametrize("k8v3", [False, True])
def test_window_tree_verify_with_fresh_drafts(k8v3):
    """Tree masks over fresh drafts (ancestor bits select the visible drafts)."""
    nq = 24
    case, cache, q, pre = _verify_case(731, 3, 16, 4, 128, 16, [1500, 600, 90], nq, k8v3)
    rng = np.random.default_rng(732)
    masks = np.zeros((3, nq), np.int64)
    for b in range(3):
        for i in range(nq):
            par = int(rng.integers(-1, i)) if i else -1
            masks[b, i] = (masks[b, par] if par >= 0 else 0) | (1 << i)
    kd, vd = _drafts(case, pre, nq)
    c = [_t(x) for x in cache]
    kw = dict(max_context_len=int(case.block_table.shape[1] * case.block_size), scale=case.scale, window=400,
              tree_mask=_t(masks), k_draft=_t(kd), v_draft=_t(vd))
    bt, pl = _t(case.block_table), _t(pre.astype(np.int32))
    if k8v3:
        out = ops.attn_paged_verify_k8v3(_t(q), *c, _t(CODEBOOK), bt, pl, case.block_size, **kw)
    else:
        out = ops.attn_paged_verify(_t(q), *c, bt, pl, case.block_size, **kw)
    layer = O.LayerCache(cache[0], cache[1], v_packed=cache[2], v_norm=cache[3], v_codebook=CODEBOOK) if k8v3 \
        else O.LayerCache(*cache)
    ref = O.paged_verify(q, layer, case.block_table, pre, case.scale, tree_mask=masks, window=400,
                         fresh_drafts=(kd, vd))
    _close(out.float().cpu().numpy(), ref, "tree verify window 400 with fresh drafts")


@pytest.mark.parametrize("k8v3", [False, True])
def test_window_verify_fresh_drafts_query_lens(k8v3):
    """Rows with fewer drafts than the call's S (query_lens, one row with
    none): their queries past the count are zeros and the drafts past it are
    never read (NaN there changes nothing); the live rows match the oracle."""
    nq = 20
    ql = np.array([20, 7, 0, 13], np.int32)
    case, cache, q, pre = _verify_case(741, 4, 16, 4, 128, 16, [900, 2500, 300, 64], nq, k8v3)
    kd, vd = _drafts(case, pre, nq)
    kd, vd = kd.copy(), vd.copy()
    for b, n in enumerate(ql):
        kd[b, n:] = np.nan
        vd[b, n:] = np.nan
    c = [_t(x) for x in cache]
    kw = dict(max_context_len=int(case.block_table.shape[1] * case.block_size), scale=case.scale, window=600,
              query_lens=_t(ql), k_draft=_t(kd), v_draft=_t(vd))
    bt, pl = _t(case.block_table), _t(pre.astype(np.int32))
    if k8v3:
        out = ops.attn_paged_verify_k8v3(_t(q), *c, _t(CODEBOOK), bt, pl, case.block_size, **kw)
    else:
        out = ops.attn_paged_verify(_t(q), *c, bt, pl, case.block_size, **kw)
    got = out.float().cpu().numpy()
    for b, n in enumerate(ql):
        assert not got[b, :, n:].any(), f"row {b}: outputs past its {n} queries"
    layer = O.LayerCache(cache[0], cache[1], v_packed=cache[2], v_norm=cache[3], v_codebook=CODEBOOK) if k8v3 \
        else O.LayerCache(*cache)
    clean_k, clean_v = _drafts(case, pre, nq)
    ref = O.paged_verify(q, layer, case.block_table, pre, case.scale, query_lens=ql, window=600,
                         fresh_drafts=(clean_k, clean_v))
    _close(got, ref, "window verify with fresh drafts and query_lens")


def test_fresh_drafts_need_a_window():
    case, cache, q, pre = _verify_case(711, 1, 8, 2, 128, 16, [100], 4)
    kd, vd = _drafts(case, pre, 4)
    with pytest.raises(ValueError):
        ops.attn_paged_verify(_t(q), *[_t(x) for x in cache], _t(case.block_table), _t(pre.astype(np.int32)),
                              case.block_size, max_context_len=128, scale=0.1, k_draft=_t(kd), v_draft=_t(vd))
