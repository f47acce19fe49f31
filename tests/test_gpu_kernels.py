"""GPU parity of the HIP kernels against the CPU oracle.

Cache bytes, scales, packed codes and norms must be bit-exact; attention
outputs must satisfy max(|out-ref| / max(1,|ref|)) <= 2e-3 and relative RMS
<= 1e-3 against the float64 oracle over the exactly dequantized cache.
All calls go through the C ABI (ctypes) of libsuperl8_kv.so.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops
from tests.kvcase import make_case, oracle_fill_int8, oracle_fill_k8v3

pytestmark = pytest.mark.gpu

DEV = "cuda"
CODEBOOK = O.gaussian_codebook(3, 128)


def _t(x, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(x))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(DEV)


def _np(t):
    return t.detach().cpu().numpy()


def _gpu_int8_cache(case):
    shape = (case.num_blocks, case.num_kv_heads, case.block_size, case.head_dim)
    return (torch.zeros(shape, dtype=torch.int8, device=DEV), torch.ones(shape[:3], dtype=torch.float32, device=DEV),
            torch.zeros(shape, dtype=torch.int8, device=DEV), torch.ones(shape[:3], dtype=torch.float32, device=DEV))


def _gpu_k8v3_cache(case):
    shape = (case.num_blocks, case.num_kv_heads, case.block_size, case.head_dim)
    d = case.head_dim
    return (torch.zeros(shape, dtype=torch.int8, device=DEV), torch.ones(shape[:3], dtype=torch.float32, device=DEV),
            torch.zeros(shape[:3] + (d * 3 // 32,), dtype=torch.int32, device=DEV),
            torch.zeros(shape[:3] + (d // 128,), dtype=torch.float32, device=DEV))


def _assert_attention_close(out, ref, what):
    mx, rel = O.attention_errors(out, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"


# ---------------------------------------------------------------------------
# append
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("d,bs,lens", [
    (128, 256, [300, 1, 17]),
    (128, 16, [33, 64, 5, 16]),
    (256, 16, [40, 3]),
    (64, 4, [9, 31]),
    (32, 8, [17, 2, 40]),
])
def test_append_int8_bitexact(d, bs, lens):
    case = make_case(10 + d + bs, len(lens), 4 * 2, 2, d, bs, lens)
    ref = oracle_fill_int8(case)
    kc, ks, vc, vs = _gpu_int8_cache(case)
    ops.quantize_kv_write_paged(_t(case.k), _t(case.v), kc, ks, vc, vs, _t(case.slots))
    torch.cuda.synchronize()
    for name, g, r in zip(("k_cache", "k_scale", "v_cache", "v_scale"), (kc, ks, vc, vs), ref):
        got = _np(g)
        assert got.dtype == r.dtype
        assert np.array_equal(got.view(np.uint8) if got.dtype == np.int8 else got.view(np.uint32),
                              r.view(np.uint8) if r.dtype == np.int8 else r.view(np.uint32)), f"{name} differs"


def test_append_int8_special_rows():
    """Zero rows, RNE ties, fp16 extremes and subnormals."""
    d, hkv, bs = 128, 2, 16
    rows = []
    rows.append(np.zeros(d))                               # zero row -> scale 0, codes 0
    r = np.zeros(d); r[0] = 127.0; r[1] = 2.5; r[2] = -2.5; r[3] = 3.5; rows.append(r)  # RNE ties
    r = np.full(d, 4096.0); r[::2] = -4096.0; rows.append(r)  # rotates to one 46341 coefficient
    r = np.full(d, 2.0 ** -24); r[5] = 2.0 ** -14; rows.append(r)  # subnormals
    r = np.linspace(-1, 1, d); rows.append(r)
    r = np.zeros(d); r[7] = -1e-3; rows.append(r)
    t = len(rows)
    k = np.stack([np.stack([x, -x]) for x in rows]).astype(np.float16)  # [t, 2, d]
    v = k[:, ::-1].copy()
    v[2, 0] = 65504.0  # V is not rotated: the fp16 extreme itself
    v[2, 1, ::3] = -65504.0
    slots = np.arange(t, dtype=np.int32) * 3
    nb = (slots.max() // bs) + 2
    shape = (nb, hkv, bs, d)
    ref = [np.zeros(shape, np.int8), np.ones(shape[:3], np.float32), np.zeros(shape, np.int8), np.ones(shape[:3], np.float32)]
    O.quantize_kv_write_paged(k, v, *ref, slots)
    g = [torch.zeros(shape, dtype=torch.int8, device=DEV), torch.ones(shape[:3], device=DEV),
         torch.zeros(shape, dtype=torch.int8, device=DEV), torch.ones(shape[:3], device=DEV)]
    ops.quantize_kv_write_paged(_t(k), _t(v), *g, _t(slots))
    for a, b in zip(g, ref):
        assert np.array_equal(_np(a), b)


@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_append_int8_input_views(d):
    """The same tokens written from contiguous K/V (several rows per wave),
    from K/V slices of a fused qkv projection output (strided, 16-byte aligned
    rows: several rows per wave) and from views 2 bytes off alignment (one row
    per wave): every cache byte equals the oracle's."""
    hq, hkv, bs = 4, 2, 16
    case = make_case(40 + d, 3, hq, hkv, d, bs, [37, 16, 70])
    ref = oracle_fill_int8(case)
    t = case.k.shape[0]
    qkv = torch.zeros((t, (hq + 2 * hkv) * d), dtype=torch.float16, device=DEV)
    qkv[:, hq * d:(hq + hkv) * d] = _t(case.k).reshape(t, hkv * d)
    qkv[:, (hq + hkv) * d:] = _t(case.v).reshape(t, hkv * d)
    k_slice = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v_slice = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    flat = torch.zeros(2 * t * hkv * d + 1, dtype=torch.float16, device=DEV)
    k_odd = flat[1:1 + t * hkv * d].view(t, hkv, d)
    v_odd = flat[1 + t * hkv * d:].view(t, hkv, d)
    k_odd.copy_(_t(case.k))
    v_odd.copy_(_t(case.v))
    assert k_slice.stride(0) == (hq + 2 * hkv) * d and k_odd.data_ptr() % 16 == 2
    for name, (kk, vv) in {"contiguous": (_t(case.k), _t(case.v)), "qkv slices": (k_slice, v_slice),
                           "unaligned": (k_odd, v_odd)}.items():
        kc, ks, vc, vs = _gpu_int8_cache(case)
        ops.quantize_kv_write_paged(kk, vv, kc, ks, vc, vs, _t(case.slots))
        torch.cuda.synchronize()
        for what, g, r in zip(("k_cache", "k_scale", "v_cache", "v_scale"), (kc, ks, vc, vs), ref):
            assert np.array_equal(_np(g).view(np.uint8), r.view(np.uint8)), f"{name}: {what} differs"


def test_append_negative_slot_skipped():
    case = make_case(3, 2, 4, 2, 128, 16, [20, 5])
    slots = case.slots.copy()
    slots[3] = -1
    slots[10] = -1
    kc0, ks0, vc0, vs0 = _gpu_int8_cache(case)
    ops.quantize_kv_write_paged(_t(case.k), _t(case.v), kc0, ks0, vc0, vs0, _t(slots))
    ref = [np.zeros((case.num_blocks, 2, 16, 128), np.int8), np.ones((case.num_blocks, 2, 16), np.float32),
           np.zeros((case.num_blocks, 2, 16, 128), np.int8), np.ones((case.num_blocks, 2, 16), np.float32)]
    O.quantize_kv_write_paged(case.k, case.v, *ref, slots)
    for a, b in zip((kc0, ks0, vc0, vs0), ref):
        assert np.array_equal(_np(a), b)


@pytest.mark.parametrize("d,bs,lens", [(128, 256, [300, 7]), (128, 16, [40, 16, 1]), (256, 16, [33, 4])])
def test_append_k8v3_bitexact(d, bs, lens):
    case = make_case(20 + d + bs, len(lens), 8, 2, d, bs, lens, outlier_channels=2)
    ref = oracle_fill_k8v3(case, CODEBOOK)
    g = _gpu_k8v3_cache(case)
    ops.quantize_kv_write_paged_k8v3(_t(case.k), _t(case.v), *g, _t(CODEBOOK), _t(case.slots))
    torch.cuda.synchronize()
    for name, a, b in zip(("k_cache", "k_scale", "v_packed", "v_norm"), g, ref):
        got = _np(a)
        assert np.array_equal(got.view(np.uint8), b.view(np.uint8)), f"{name} differs"


@pytest.mark.parametrize("d", [128, 256])
def test_append_k8v3_input_views(d):
    """K8V3 writes from 16-byte aligned rows (several rows per wave) and from
    views 2 bytes off alignment (one row per wave): both equal the oracle."""
    hkv, bs = 2, 16
    case = make_case(50 + d, 3, 4, hkv, d, bs, [37, 16, 70], outlier_channels=2)
    ref = oracle_fill_k8v3(case, CODEBOOK)
    t = case.k.shape[0]
    flat = torch.zeros(2 * t * hkv * d + 1, dtype=torch.float16, device=DEV)
    k_odd = flat[1:1 + t * hkv * d].view(t, hkv, d)
    v_odd = flat[1 + t * hkv * d:].view(t, hkv, d)
    k_odd.copy_(_t(case.k))
    v_odd.copy_(_t(case.v))
    for name, (kk, vv) in {"aligned": (_t(case.k), _t(case.v)), "unaligned": (k_odd, v_odd)}.items():
        g = _gpu_k8v3_cache(case)
        ops.quantize_kv_write_paged_k8v3(kk, vv, *g, _t(CODEBOOK), _t(case.slots))
        torch.cuda.synchronize()
        for what, a, b in zip(("k_cache", "k_scale", "v_packed", "v_norm"), g, ref):
            assert np.array_equal(_np(a).view(np.uint8), b.view(np.uint8)), f"{name}: {what} differs"


@pytest.mark.parametrize("kind", ["permuted", "wide", "repeated"])
def test_append_k8v3_codebook_outside_search_condition(kind):
    """Codebooks the three-comparison search does not accept (not ascending,
    entries beyond +-4, a repeated entry) take the sequential scan: the bytes
    still equal the oracle's first-minimum codes, from aligned and unaligned
    inputs."""
    cb = CODEBOOK.copy()
    if kind == "permuted":
        cb = cb[[3, 0, 6, 1, 7, 2, 5, 4]]
    elif kind == "wide":
        cb = (cb * 40.0).astype(np.float32)
    else:
        cb[5] = cb[4]
    d, hkv, bs = 128, 2, 16
    case = make_case(77, 2, 4, hkv, d, bs, [40, 9], outlier_channels=2)
    ref = oracle_fill_k8v3(case, cb)
    t = case.k.shape[0]
    flat = torch.zeros(2 * t * hkv * d + 1, dtype=torch.float16, device=DEV)
    k_odd = flat[1:1 + t * hkv * d].view(t, hkv, d)
    v_odd = flat[1 + t * hkv * d:].view(t, hkv, d)
    k_odd.copy_(_t(case.k))
    v_odd.copy_(_t(case.v))
    for name, (kk, vv) in {"aligned": (_t(case.k), _t(case.v)), "unaligned": (k_odd, v_odd)}.items():
        g = _gpu_k8v3_cache(case)
        ops.quantize_kv_write_paged_k8v3(kk, vv, *g, _t(cb), _t(case.slots))
        torch.cuda.synchronize()
        for what, a, b in zip(("k_cache", "k_scale", "v_packed", "v_norm"), g, ref):
            assert np.array_equal(_np(a).view(np.uint8), b.view(np.uint8)), f"{kind} {name}: {what} differs"


def test_append_k8v3_zero_and_tie_rows():
    d, hkv, bs = 128, 1, 4
    rows = [np.zeros(d), np.ones(d), np.r_[np.ones(64), -np.ones(64)], np.linspace(-3, 3, d)]
    v = np.stack(rows)[:, None, :].astype(np.float16)
    k = v.copy()
    slots = np.arange(len(rows), dtype=np.int32)
    shape = (1, hkv, bs, d)
    ref = [np.zeros(shape, np.int8), np.ones(shape[:3], np.float32), np.zeros(shape[:3] + (12,), np.int32),
           np.zeros(shape[:3] + (1,), np.float32)]
    O.k8v3_write_paged(k, v, *ref, CODEBOOK, slots)
    g = [torch.zeros(shape, dtype=torch.int8, device=DEV), torch.ones(shape[:3], device=DEV),
         torch.zeros(shape[:3] + (12,), dtype=torch.int32, device=DEV), torch.zeros(shape[:3] + (1,), device=DEV)]
    ops.quantize_kv_write_paged_k8v3(_t(k), _t(v), *g, _t(CODEBOOK), _t(slots))
    for a, b in zip(g, ref):
        assert np.array_equal(_np(a).view(np.uint8), b.view(np.uint8))


# ---------------------------------------------------------------------------
# decode
# ---------------------------------------------------------------------------


def _decode_gpu_int8(case, cache, **kw):
    kc, ks, vc, vs = (_t(x) for x in cache)
    q = _t(case.q)[:, :, None, :]
    out = ops.attn_paged_decode_cached(q, kc, ks, vc, vs, _t(case.block_table), _t(case.lens.astype(np.int32)),
                                       case.block_size, max_context_len=int(case.lens.max()), scale=case.scale, **kw)
    return _np(out.float())[:, :, 0, :]


def _decode_ref(case, cache, k8v3=False):
    if k8v3:
        kc, ks, vp, vn = cache
        layer = O.LayerCache(kc, ks, v_packed=vp, v_norm=vn, v_codebook=CODEBOOK)
    else:
        kc, ks, vc, vs = cache
        layer = O.LayerCache(kc, ks, vc, vs)
    return O.paged_decode(case.q, layer, case.block_table, case.lens, case.scale)


@pytest.mark.parametrize("hq,hkv,d,bs,lens", [
    (16, 8, 128, 256, [129, 1024, 300, 1]),          # Qwen3-0.6B-shaped, bs 256
    (32, 8, 128, 256, [2049, 31, 32, 33]),           # Qwen3-8B heads
    (32, 8, 128, 16, [100, 17, 16, 15, 1]),          # reference default block size
    (8, 8, 128, 16, [45, 64]),                       # no GQA
    (16, 1, 128, 32, [70]),                          # 16 q heads on one kv head
    (8, 2, 256, 16, [50, 129]),
    (8, 4, 64, 8, [33, 2, 80]),
    (4, 2, 32, 4, [9, 31, 12]),
])
def test_decode_int8_vs_oracle(hq, hkv, d, bs, lens):
    case = make_case(1000 + hq + d + bs, len(lens), hq, hkv, d, bs, lens)
    cache = oracle_fill_int8(case)
    got = _decode_gpu_int8(case, cache)
    ref = _decode_ref(case, cache)
    _assert_attention_close(got, ref, "decode")


def test_decode_int8_outlier_channels():
    """1% outlier channels scaled 20x on q, K and V (the 8B workload's data)."""
    case = make_case(7, 6, 32, 8, 128, 256, [2048, 700, 4096, 256, 1500, 33], outlier_channels=2)
    cache = oracle_fill_int8(case)
    _assert_attention_close(_decode_gpu_int8(case, cache), _decode_ref(case, cache), "decode outliers")


@pytest.mark.parametrize(
    "wg_per_head,ghost,batch,hq,hkv,bs,lens,skew",
    [
        # one workgroup per head: every row in one slice, rows past 2048 tokens
        # streamed in several block-id stages
        (1, 128, 4, 16, 4, 16, [1000, 129, 5000, 0], 0),
        # slices longer than 2048 tokens that end inside a row
        (2, 0, 4, 8, 2, 256, [5000, 100, 0, 37], 0),
        # many short rows: slices span several rows, rows span slices
        (7, 0, 64, 32, 8, 32, "short", 0),
        (7, 128, 64, 32, 8, 32, "short", 0),
        # per-row charge larger than the slices: some slices hold no tokens
        (40, 512, 64, 32, 8, 16, "short", 0),
        # block_size < 32: tiles cross blocks
        (3, 64, 5, 16, 4, 8, [300, 1, 64, 2500, 31], 0),
        # slices weighted by residency slot (unequal slice lengths)
        (7, 256, 64, 32, 8, 32, "short", 300),
        (5, 0, 4, 8, 2, 256, [5000, 100, 0, 3000], 150),
    ],
)
def test_decode_int8_slicings(wg_per_head, ghost, batch, hq, hkv, bs, lens, skew, monkeypatch):
    """Other slicings of the token stream across workgroups: whole rows, rows
    split across slices (partials + merge), slices spanning several rows, and
    slices that fall between rows' tokens."""
    monkeypatch.setenv("S8KV_DECODE_WG_PER_HEAD", str(wg_per_head))
    monkeypatch.setenv("S8KV_DECODE_GHOST", str(ghost))
    monkeypatch.setenv("S8KV_DECODE_SLOT_SKEW", str(skew))
    if lens == "short":
        lens = np.random.default_rng(5).integers(0, 120, size=batch).tolist()
    case = make_case(55 + wg_per_head, batch, hq, hkv, 128, bs, lens)
    cache = oracle_fill_int8(case)
    _assert_attention_close(_decode_gpu_int8(case, cache), _decode_ref(case, cache), f"decode wg/head={wg_per_head}")


def test_decode_q_transpose_view():
    """The attention seam passes q as a [B,1,H,D] -> [B,H,1,D] transpose view
    (gqa_attention.py:168-172)."""
    case = make_case(77, 3, 8, 2, 128, 16, [40, 7, 64])
    cache = oracle_fill_int8(case)
    kc, ks, vc, vs = (_t(x) for x in cache)
    hq, hkv, d = 8, 2, 128
    qkv = torch.zeros((3, 1, (hq + 2 * hkv) * d), dtype=torch.float16, device=DEV)
    qkv[:, 0, : hq * d] = _t(case.q).reshape(3, hq * d)
    q_view = qkv[..., : hq * d].view(3, 1, hq, d).transpose(1, 2)  # [B,H,1,D] strided view
    assert q_view.stride(0) == (hq + 2 * hkv) * d and q_view.stride(1) == d
    out = ops.attn_paged_decode_cached(q_view, kc, ks, vc, vs, _t(case.block_table), _t(case.lens.astype(np.int32)),
                                       16, max_context_len=64, scale=case.scale)
    _assert_attention_close(_np(out.float())[:, :, 0], _decode_ref(case, cache), "transpose view")


def test_decode_max_context_len_is_only_a_bound():
    case = make_case(78, 2, 8, 2, 128, 16, [20, 3], width=16)
    cache = oracle_fill_int8(case)
    ref = _decode_ref(case, cache)
    kc, ks, vc, vs = (_t(x) for x in cache)
    for mcl in (20, 128, 256):
        out = ops.attn_paged_decode_cached(_t(case.q)[:, :, None], kc, ks, vc, vs, _t(case.block_table),
                                           _t(case.lens.astype(np.int32)), 16, max_context_len=mcl, scale=case.scale)
        _assert_attention_close(_np(out.float())[:, :, 0], ref, f"max_context_len={mcl}")


@pytest.mark.parametrize("d,bs,lens", [(128, 256, [300, 1, 1024]), (128, 16, [47, 16]), (256, 16, [70, 9])])
def test_decode_k8v3_vs_oracle(d, bs, lens):
    case = make_case(500 + d + bs, len(lens), 8, 2, d, bs, lens)
    cache = oracle_fill_k8v3(case, CODEBOOK)
    kc, ks, vp, vn = (_t(x) for x in cache)
    out = ops.attn_paged_decode_k8v3(_t(case.q)[:, :, None], kc, ks, vp, vn, _t(CODEBOOK), _t(case.block_table),
                                     _t(case.lens.astype(np.int32)), bs, max_context_len=int(max(lens)),
                                     scale=case.scale)
    _assert_attention_close(_np(out.float())[:, :, 0], _decode_ref(case, cache, k8v3=True), "decode k8v3")


def test_end_to_end_append_then_decode_c1():
    """Qwen3-0.6B-shaped single-layer step: B=8, L ~ U[128,1024] prefill, one
    appended token per row, 16 q / 8 kv heads, D=128, bs=256, seed 0."""
    rng = np.random.default_rng(0)
    prefill = rng.integers(128, 1025, 8)
    lens = prefill + 1
    case = make_case(0, 8, 16, 8, 128, 256, lens)
    ref_cache = oracle_fill_int8(case)
    kc, ks, vc, vs = _gpu_int8_cache(case)
    # prefill (varlen) then the decode append, in two calls like the engine
    first = np.concatenate([np.arange(int(lens[:b].sum()), int(lens[:b].sum()) + int(prefill[b])) for b in range(8)])
    last = np.array([int(lens[: b + 1].sum()) - 1 for b in range(8)])
    ops.quantize_kv_write_paged(_t(case.k[first]), _t(case.v[first]), kc, ks, vc, vs, _t(case.slots[first]))
    ops.quantize_kv_write_paged(_t(case.k[last]), _t(case.v[last]), kc, ks, vc, vs, _t(case.slots[last]))
    for g, r in zip((kc, ks, vc, vs), ref_cache):
        assert np.array_equal(_np(g), r)
    out = ops.attn_paged_decode_cached(_t(case.q)[:, :, None], kc, ks, vc, vs, _t(case.block_table),
                                       _t(lens.astype(np.int32)), 256, max_context_len=int(lens.max()),
                                       scale=case.scale)
    _assert_attention_close(_np(out.float())[:, :, 0], _decode_ref(case, ref_cache), "C1")


# ---------------------------------------------------------------------------
# block copy
# ---------------------------------------------------------------------------


def test_copy_blocks_bitexact():
    rng = np.random.default_rng(5)
    nl, nb, hkv, bs, d = 3, 12, 2, 16, 128
    tens = [rng.integers(-127, 128, (nl, nb, hkv, bs, d)).astype(np.int8),
            rng.standard_normal((nl, nb, hkv, bs)).astype(np.float32),
            rng.integers(-2**31, 2**31 - 1, (nl, nb, hkv, bs, 12), dtype=np.int64).astype(np.int32),
            rng.standard_normal((nl, nb, hkv, bs, 1)).astype(np.float32)]
    src, dst = [1, 5, 7], [0, 11, 3]
    gpu = [_t(x) for x in tens]
    ops.copy_blocks(gpu, src, dst)
    O.copy_blocks(tens, src, dst)
    for a, b in zip(gpu, tens):
        assert np.array_equal(_np(a), b)
    with pytest.raises(ValueError):
        ops.copy_blocks(gpu, [1], [1])


def test_copy_blocks_odd_block_bytes():
    """Blocks whose byte size is not a multiple of 16 (tiny test geometries)."""
    rng = np.random.default_rng(6)
    x = rng.standard_normal((2, 9, 1, 5)).astype(np.float32)  # 20-byte blocks
    g = _t(x)
    ops.copy_blocks([g], [8, 2], [0, 4])
    O.copy_blocks([x], [8, 2], [0, 4])
    assert np.array_equal(_np(g), x)


def test_copy_blocks_multi_chunk_and_unaligned_base():
    """10,560-byte blocks (two workgroup chunks, the second partial), once in
    a 16-byte aligned tensor (vector path) and once in a contiguous view that
    starts 4 bytes into its storage (word path)."""
    rng = np.random.default_rng(7)
    shape = (2, 7, 5, 33, 64)
    x = rng.integers(-128, 128, shape).astype(np.int8)
    src, dst = [6, 1, 3], [0, 5, 2]
    ref = x.copy()
    O.copy_blocks([ref], src, dst)
    g = _t(x)
    ops.copy_blocks([g], src, dst)
    assert np.array_equal(_np(g), ref)
    buf = torch.zeros(x.size + 4, dtype=torch.int8, device=DEV)
    v = buf[4:].view(shape)
    assert v.is_contiguous() and v.data_ptr() % 16 == 4
    v.copy_(torch.from_numpy(x).to(DEV))
    ops.copy_blocks([v], src, dst)
    assert np.array_equal(_np(v), ref)
    assert int(buf[:4].abs().sum()) == 0


# ---------------------------------------------------------------------------
# HIP graph capture
# ---------------------------------------------------------------------------


def test_graph_capture_append_and_decode():
    """Append + decode captured in a graph, replayed with fresh inputs copied
    into the static buffers; every replay equals the eager result."""
    case = make_case(90, 4, 8, 2, 128, 16, [60, 33, 5, 17], spare_blocks=8)
    base = oracle_fill_int8(case)
    kc, ks, vc, vs = (_t(x) for x in base)
    bt = _t(case.block_table)
    cl = _t(case.lens.astype(np.int32))
    slots = _t(case.slots[:4])
    k_in = torch.zeros((4, 2, 128), dtype=torch.float16, device=DEV)
    v_in = torch.zeros_like(k_in)
    q_in = torch.zeros((4, 8, 1, 128), dtype=torch.float16, device=DEV)

    def step():
        ops.quantize_kv_write_paged(k_in, v_in, kc, ks, vc, vs, slots)
        return ops.attn_paged_decode_cached(q_in, kc, ks, vc, vs, bt, cl, 16, max_context_len=64, scale=case.scale)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = step()
    rng = np.random.default_rng(91)
    for rep in range(3):
        kx = torch.from_numpy(rng.standard_normal((4, 2, 128)).astype(np.float16)).to(DEV)
        vx = torch.from_numpy(rng.standard_normal((4, 2, 128)).astype(np.float16)).to(DEV)
        qx = torch.from_numpy(rng.standard_normal((4, 8, 1, 128)).astype(np.float16)).to(DEV)
        k_in.copy_(kx); v_in.copy_(vx); q_in.copy_(qx)
        graph.replay()
        torch.cuda.synchronize()
        got = out_static.clone()
        eager = step()
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {rep} differs from eager"
