"""Pins the CPU oracle before it is trusted as the GPU kernels' checker.

Each oracle function is checked against something independent of it:
published tables (Max 1960), library routines (scipy's Hadamard), exact
known-answer vectors computed by integer / rational arithmetic
(tests/golden/make_known_answers.py), the reference's own tests' quality bars
and exact byte counts, closed forms and invariants (involution, chain verify
== sequential decodes, block relocation leaves every read unchanged), and an
independent float64 torch restatement of the attention.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import scipy.integrate
import scipy.linalg
import scipy.stats
import torch

from oracle import kv_oracle as O

GOLD = json.loads((Path(__file__).resolve().parent / "golden" / "known_answers.json").read_text())


def _cos(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def _sqnr_db(ref, q):
    ref = np.asarray(ref, np.float64)
    err = ref - np.asarray(q, np.float64)
    return float(10 * np.log10((ref * ref).sum() / (err * err).sum()))


# ---------------------------------------------------------------------------
# Hadamard rotation
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("d", [2, 4, 8, 16, 32, 64, 128, 256])
def test_hadamard_is_normalized_sylvester(d):
    h = O.hadamard_matrix(d)
    assert np.array_equal(h * math.sqrt(d), scipy.linalg.hadamard(d).astype(np.float64))
    assert np.allclose(h, h.T) and np.allclose(h @ h, np.eye(d), atol=1e-12)  # involution (kv_cache.py:274-277)


@pytest.mark.parametrize("case", GOLD["fwht"], ids=lambda c: f"n{len(c['x'])}")
def test_fwht_known_answers(case):
    x = np.asarray(case["x"], np.float32)
    assert np.array_equal(O.fwht_f32(x), np.asarray(case["y"], np.float32))


def test_fwht_batched_axes_and_basis_vectors():
    d = 64
    eye = np.eye(d, dtype=np.float32)
    assert np.array_equal(O.fwht_f32(eye), scipy.linalg.hadamard(d).astype(np.float32))
    x = np.random.default_rng(0).integers(-9, 10, size=(3, 5, d)).astype(np.float32)
    ref = x.astype(np.float64) @ scipy.linalg.hadamard(d)
    assert np.array_equal(O.fwht_f32(x), ref.astype(np.float32))


def test_rotate_last_matches_matrix_and_is_involution():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((50, 4, 128)).astype(np.float16)
    y = O.rotate_last(x)
    assert y.dtype == np.float16
    ref = x.astype(np.float64) @ O.hadamard_matrix(128)
    # one fp16 rounding of a value computed in fp32: within 1 fp16 ulp
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(y.astype(np.float64) - ref) <= ulp)
    back = O.rotate_last(y)
    assert np.max(np.abs(back.astype(np.float64) - x.astype(np.float64))) < 4e-3


# ---------------------------------------------------------------------------
# int8 RTN
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("i", range(len(GOLD["rtn_int8"])))
def test_rtn_known_answers(i):
    case = GOLD["rtn_int8"][i]
    q, s = O.quantize_i8_rowwise(np.asarray([case["x"]], np.float32))
    assert s.dtype == np.float32 and q.dtype == np.int8
    assert s[0] == np.float32(case["scale"])
    assert q[0].tolist() == case["codes"]


def test_rtn_rules():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((200, 128)) * rng.uniform(1e-3, 1e3, (200, 1))).astype(np.float32)
    q, s = O.quantize_i8_rowwise(x)
    assert np.all(np.abs(q.astype(np.int32)).max(axis=1) == 127)  # absmax element maps to +-127
    err = np.abs(O.dequantize_int8_rowwise(q, s).astype(np.float64) - x)
    assert np.all(err <= s[:, None].astype(np.float64) * 0.5 * (1 + 1e-6))


def test_k_quality_bar_of_reference():
    """int8 K after rotation: cos >= 0.999 and SQNR >= 35 dB
    (tests/test_k8v3_cache.py:113-121)."""
    rng = np.random.default_rng(7)
    k = rng.standard_normal((2, 4, 8, 256)).astype(np.float16)
    kr = O.rotate_last(k)
    q, s = O.quantize_i8_rowwise(kr)
    deq = O.dequantize_int8_rowwise(q, s)
    assert _cos(kr, deq) >= 0.999 and _sqnr_db(kr, deq) >= 35.0


# ---------------------------------------------------------------------------
# Paged layout and append
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("case", GOLD["flat_rows"], ids=lambda c: f"h{c['num_kv_heads']}bs{c['block_size']}")
def test_flat_rows_known_answers(case):
    rows = O.flat_rows(np.asarray(case["slots"]), case["num_kv_heads"], case["block_size"])
    assert rows.tolist() == case["rows"]


def test_append_writes_exactly_the_mapped_rows():
    rng = np.random.default_rng(3)
    n, hkv, bs, d = 6, 2, 4, 32
    k = rng.standard_normal((5, hkv, d)).astype(np.float16)
    v = rng.standard_normal((5, hkv, d)).astype(np.float16)
    slots = np.array([0, 7, -1, 13, 22], np.int32)
    shape = (n, hkv, bs, d)
    kc, vc = np.full(shape, 99, np.int8), np.full(shape, 99, np.int8)
    ks, vs = np.full(shape[:3], 5.0, np.float32), np.full(shape[:3], 5.0, np.float32)
    O.quantize_kv_write_paged(k, v, kc, ks, vc, vs, slots)
    written = np.zeros(shape[:3], bool)
    for t, sl in enumerate(slots):
        if sl < 0:
            continue
        blk, off = sl // bs, sl % bs
        for h in range(hkv):
            written[blk, h, off] = True
            qk, sk = O.quantize_i8_rowwise(O.rotate_last(k[t, h]))
            qv, sv = O.quantize_i8_rowwise(v[t, h])
            assert np.array_equal(kc[blk, h, off], qk) and ks[blk, h, off] == sk
            assert np.array_equal(vc[blk, h, off], qv) and vs[blk, h, off] == sv
    assert np.all(kc[~written] == 99) and np.all(ks[~written] == 5.0)
    assert np.all(vc[~written] == 99) and np.all(vs[~written] == 5.0)


@pytest.mark.parametrize("case", GOLD["block_bytes"], ids=lambda c: f"{c['v_quant']}-{c['block_size']}-{c['head_dim']}")
def test_block_bytes(case):
    got = O.block_bytes(case["num_kv_heads"], case["block_size"], case["head_dim"], case["v_quant"])
    assert got == case["bytes"]


def test_block_bytes_reference_envelope():
    """The reference's 262k-context K8V3 envelope: 16 layers x 262144 tokens at
    4 KV heads, head_dim 256, block 16 is 5.5..6.5 GiB
    (tests/test_k8v3_cache.py:567-575)."""
    bb = O.block_bytes(4, 16, 256, "lloydmax3")
    assert 5.5 <= 16 * (262144 // 16) * bb / 2**30 <= 6.5
    assert bb < O.block_bytes(4, 16, 256, "int8")


# ---------------------------------------------------------------------------
# K8V3 V codec
# ---------------------------------------------------------------------------


def test_lloyd_max_levels_match_max_1960():
    lv = O.lloyd_max_gaussian_levels(8)
    pos = lv[4:]
    assert np.allclose(lv, -lv[::-1], atol=1e-12)  # odd symmetric
    assert np.allclose(pos, GOLD["max1960"]["levels"], atol=1.5e-4)
    ends = 0.5 * (lv[1:] + lv[:-1])
    assert np.allclose(ends[3:], GOLD["max1960"]["thresholds"], atol=1.5e-4)


def test_lloyd_max_centroid_condition():
    """Every level is the conditional mean of N(0,1) over its cell (the
    necessary condition of a minimum-MSE quantizer), by numerical quadrature."""
    lv = O.lloyd_max_gaussian_levels(8)
    edges = np.concatenate([[-np.inf], 0.5 * (lv[1:] + lv[:-1]), [np.inf]])
    for i in range(8):
        a, b = edges[i], edges[i + 1]
        num = scipy.integrate.quad(lambda x: x * scipy.stats.norm.pdf(x), a, b)[0]
        den = scipy.stats.norm.cdf(b) - scipy.stats.norm.cdf(a)
        assert abs(num / den - lv[i]) < 1e-9


def test_gaussian_codebook():
    cb = O.gaussian_codebook(3, 128)
    assert cb.dtype == np.float32 and cb.shape == (8,)
    assert np.all(np.diff(cb) > 0)
    assert np.array_equal(cb, (O.lloyd_max_gaussian_levels(8) / math.sqrt(128)).astype(np.float32))


def test_l2_norm_blocks():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((40, 256)).astype(np.float16)
    n = O.l2_norm_blocks(x, 128)
    ref = np.linalg.norm(x.astype(np.float64).reshape(40, 2, 128), axis=-1)
    assert n.dtype == np.float32 and np.allclose(n, ref, rtol=2e-7)


def test_l2_norm_blocks_summation_order():
    """The squares are added by a pairwise tree over neighbours.  With 4096
    at index 0 and ones at 64..127 every partial sum of that tree is exact
    (2^24 + 64), while folding halves (s[:h] + s[h:]) absorbs two of the ones
    into 2^24 by ties to even (2^24 + 62) and a left-to-right scan all of them
    (2^24): three different fp32 norms."""
    x = np.zeros((1, 128), np.float16)
    x[0, 0] = 4096.0
    x[0, 64:] = 1.0
    n = O.l2_norm_blocks(x, 128)[0, 0]
    want = np.float32(math.sqrt(2.0 ** 24 + 64))
    assert n == want
    assert want != np.float32(math.sqrt(2.0 ** 24 + 62)) and want != np.float32(4096.0)
    # the same block in the second half of a 256-wide row, after a zero block
    y = np.concatenate([np.zeros((1, 128), np.float16), x], axis=1)
    assert O.l2_norm_blocks(y, 128)[0].tolist() == [0.0, float(want)]


def test_quantize_lloydmax_is_nearest_codeword():
    rng = np.random.default_rng(5)
    cb = O.gaussian_codebook()
    v = rng.standard_normal((30, 256)).astype(np.float16)
    codes, norms = O.quantize_lloydmax(v, cb)
    u = v.astype(np.float32).reshape(30, 2, 128) / norms[..., None]
    dist = np.abs(u.reshape(30, 256)[..., None] - cb.astype(np.float32))
    best = dist.min(axis=-1)
    assert np.array_equal(dist[np.arange(30)[:, None], np.arange(256)[None, :], codes], best)


def test_quantize_lloydmax_zero_block():
    """A zero-norm block stores norm 0 and the first nearest code of u = 0
    (index 3: -0.2451/sqrt(128) and +0.2451/sqrt(128) tie) and dequantizes to
    exact zeros -- finite, as tests/test_k8v3_cache.py:98-111 requires."""
    v = np.zeros((2, 256), np.float16)
    v[1, 128:] = 1.0
    codes, norms = O.quantize_lloydmax(v, O.gaussian_codebook())
    assert norms[0].tolist() == [0.0, 0.0] and norms[1, 0] == 0.0
    assert np.all(codes[0] == 3) and np.all(codes[1, :128] == 3)
    deq = O.dequantize_lloydmax(codes, norms, O.gaussian_codebook())
    assert np.all(deq[0] == 0.0) and np.all(np.isfinite(deq))


def test_v_quality_bar_of_reference():
    """3-bit Lloyd-Max V on Gaussian data: cos >= 0.97 and SQNR >= 12 dB
    (tests/test_k8v3_cache.py:88-96)."""
    rng = np.random.default_rng(5)
    v = rng.standard_normal((2, 4, 16, 256)).astype(np.float16)
    cb = O.gaussian_codebook()
    codes, norms = O.quantize_lloydmax(v, cb)
    deq = O.dequantize_lloydmax(codes, norms, cb)
    assert _cos(v, deq) >= 0.97 and _sqnr_db(v, deq) >= 12.0


@pytest.mark.parametrize("i", range(len(GOLD["pack3"])))
def test_pack3_known_answers(i):
    case = GOLD["pack3"][i]
    codes = np.asarray([case["codes"]], np.uint8)
    words = O.pack_indices_lowbit(codes, 3)
    assert words.dtype == np.int32 and words[0].tolist() == case["words"]
    assert np.array_equal(O.unpack_indices_lowbit(words, 3, codes.shape[-1]), codes)


def test_pack3_roundtrip_lossless():
    codes = np.random.default_rng(6).integers(0, 8, size=(3, 5, 256)).astype(np.uint8)
    packed = O.pack_indices_lowbit(codes, 3)
    assert packed.shape == (3, 5, 256 * 3 // 32)
    assert np.array_equal(O.unpack_indices_lowbit(packed, 3, 256), codes)


# ---------------------------------------------------------------------------
# Attention oracles
# ---------------------------------------------------------------------------


def _case(seed, hkv=2, bs=8, d=64, lens=(13, 1, 40), k8v3=False, spare=3):
    rng = np.random.default_rng(seed)
    need = [-(-n // bs) for n in lens]
    nblk = sum(need) + spare
    perm = rng.permutation(nblk)
    bt = np.zeros((len(lens), max(need)), np.int32)
    pos = 0
    for b, nb in enumerate(need):
        bt[b, :nb] = perm[pos:pos + nb]
        pos += nb
    slots = np.concatenate([bt[b, np.arange(n) // bs] * bs + np.arange(n) % bs for b, n in enumerate(lens)])
    k = rng.standard_normal((len(slots), hkv, d)).astype(np.float16)
    v = rng.standard_normal((len(slots), hkv, d)).astype(np.float16)
    shape = (nblk, hkv, bs, d)
    kc, ks = np.zeros(shape, np.int8), np.ones(shape[:3], np.float32)
    if k8v3:
        vp = np.zeros(shape[:3] + (d * 3 // 32,), np.int32)
        vn = np.zeros(shape[:3] + (d // 128,), np.float32)
        cb = O.gaussian_codebook()
        O.k8v3_write_paged(k, v, kc, ks, vp, vn, cb, slots.astype(np.int32))
        layer = O.LayerCache(kc, ks, v_packed=vp, v_norm=vn, v_codebook=cb)
    else:
        vc, vs = np.zeros(shape, np.int8), np.ones(shape[:3], np.float32)
        O.quantize_kv_write_paged(k, v, kc, ks, vc, vs, slots.astype(np.int32))
        layer = O.LayerCache(kc, ks, vc, vs)
    return layer, bt, np.asarray(lens, np.int64), rng


def _torch_decode(q, layer, bt, lens, scale):
    """Independent float64 restatement: walk the positions one by one,
    dequantize with torch, un-rotate K with an explicit Sylvester matrix."""
    d = layer.head_dim
    hkv, bs = layer.num_kv_heads, layer.block_size
    hmat = torch.tensor(scipy.linalg.hadamard(d), dtype=torch.float64) / math.sqrt(d)
    qt = torch.tensor(np.asarray(q, np.float64))
    out = torch.zeros_like(qt)
    g = qt.shape[1] // hkv
    for b in range(qt.shape[0]):
        n = int(lens[b])
        if n == 0:
            continue
        for h in range(hkv):
            ks, vs = [], []
            for p in range(n):
                blk, off = int(bt[b, p // bs]), p % bs
                kr = torch.tensor(layer.k_cache[blk, h, off], dtype=torch.float64) * float(layer.k_scale[blk, h, off])
                ks.append(hmat @ kr)
                if layer.is_k8v3:
                    codes = O.unpack_indices_lowbit(layer.v_packed[blk, h, off], 3, d).astype(np.int64)
                    cb = torch.tensor(layer.v_codebook, dtype=torch.float64)[torch.tensor(codes)]
                    nrm = torch.tensor(layer.v_norm[blk, h, off], dtype=torch.float64).repeat_interleave(128)
                    vs.append(cb * nrm)
                else:
                    vs.append(torch.tensor(layer.v_cache[blk, h, off], dtype=torch.float64)
                              * float(layer.v_scale[blk, h, off]))
            kk, vv = torch.stack(ks), torch.stack(vs)
            qq = qt[b, h * g:(h + 1) * g]
            out[b, h * g:(h + 1) * g] = torch.softmax(qq @ kk.T * scale, dim=-1) @ vv
    return out.numpy()


@pytest.mark.parametrize("k8v3,d", [(False, 64), (True, 128), (True, 256)])
def test_paged_decode_matches_independent_torch(k8v3, d):
    """Against a per-position torch walk; K8V3 at head_dim 256 pins the
    norm of each 128-element block to its own half of the row."""
    layer, bt, lens, rng = _case(11, d=d, lens=(13, 1, 40, 0), k8v3=k8v3)
    q = rng.standard_normal((4, 6, d)).astype(np.float16)
    got = O.paged_decode(q, layer, bt, lens, 0.125)
    ref = _torch_decode(q, layer, bt, lens, 0.125)
    assert np.allclose(got, ref, rtol=0, atol=1e-12)
    assert np.all(got[3] == 0.0)  # empty row -> zeros


def test_paged_decode_closed_forms():
    layer, bt, lens, rng = _case(12, lens=(1, 9))
    _, v = O.exact_kv(layer, bt[0], 1)
    q = rng.standard_normal((2, 4, 64))
    out = O.paged_decode(q, layer, bt, lens, 0.3)
    assert np.allclose(out[0], np.repeat(v[:, 0], 2, axis=0), atol=1e-15)  # one key: softmax weight 1
    _, v9 = O.exact_kv(layer, bt[1], 9)
    out0 = O.paged_decode(np.zeros((2, 4, 64)), layer, bt, lens, 0.3)
    assert np.allclose(out0[1], np.repeat(v9.mean(axis=1), 2, axis=0), atol=1e-13)  # q = 0: mean of V


def test_read_dense_is_rounded_exact_kv():
    layer, bt, lens, _ = _case(13, lens=(30,))
    k16, v16 = O.read_dense(layer, bt[0], 30)
    k64, v64 = O.exact_kv(layer, bt[0], 30)
    assert k16.dtype == np.float16
    assert np.max(np.abs(k16[0].astype(np.float64) - k64)) <= np.max(np.abs(k64)) * 2e-3
    assert np.array_equal(v16[0], v64.astype(np.float32).astype(np.float16))


def test_verify_chain_equals_sequential_decodes():
    """Chain verify == S decodes with context L+t+1 (gqa_attention.py:259-277)."""
    layer, bt, lens, rng = _case(14, lens=(20, 33))
    s = 5
    prefix = lens - s
    q = rng.standard_normal((2, 4, s, 64))
    out = O.paged_verify(q, layer, bt, prefix, 0.2)
    for t in range(s):
        dec = O.paged_decode(q[:, :, t], layer, bt, prefix + t + 1, 0.2)
        assert np.allclose(out[:, :, t], dec, atol=1e-13)


def test_verify_tree_mask():
    """Tree verify: a node sees the prefix, its ancestors and itself.  A tree
    whose nodes see only themselves equals per-node decodes over prefix+node;
    query_lens beyond the row produce zeros."""
    layer, bt, lens, rng = _case(15, lens=(24,))
    p, n = 20, 4
    q = rng.standard_normal((1, 4, n, 64))
    own = np.array([[1 << i for i in range(n)]], np.int64)
    out = O.paged_verify(q, layer, bt, np.array([p]), 0.2, tree_mask=own)
    hkv, bs, d = layer.num_kv_heads, layer.block_size, layer.head_dim
    k, v = O.exact_kv(layer, bt[0], p + n)
    for i in range(n):
        idx = list(range(p)) + [p + i]
        for hh in range(4):
            h = hh // 2
            ref = O._softmax_attend(q[0, hh, i:i + 1], k[h][idx], v[h][idx], 0.2)
            assert np.allclose(out[0, hh, i], ref[0], atol=1e-13)
    part = O.paged_verify(q, layer, bt, np.array([p]), 0.2, query_lens=np.array([2]))
    assert np.all(part[0, :, 2:] == 0.0)


def test_copy_blocks_relocation_keeps_reads():
    layer, bt, lens, _ = _case(16, lens=(17, 9), spare=8)
    before = [O.read_dense(layer, bt[b], int(lens[b])) for b in range(2)]
    used = sorted(set(bt[0, :3].tolist()) | set(bt[1, :2].tolist()))
    free = [i for i in range(layer.k_cache.shape[0]) if i not in used][: len(used)]
    mapping = dict(zip(used, free))
    tensors = [t[None] for t in (layer.k_cache, layer.k_scale, layer.v_cache, layer.v_scale)]
    O.copy_blocks(tensors, used, free)
    bt2 = np.vectorize(lambda x: mapping.get(int(x), int(x)))(bt).astype(np.int32)
    for b in range(2):
        after = O.read_dense(layer, bt2[b], int(lens[b]))
        assert all(np.array_equal(x, y) for x, y in zip(before[b], after))
    with pytest.raises(ValueError):
        O.copy_blocks(tensors, [0, 1], [1, 2])


def test_attention_errors_definition():
    ref = np.array([0.5, -4.0, 10.0])
    out = np.array([0.501, -4.004, 10.0])
    mx, rel = O.attention_errors(out, ref)
    assert abs(mx - 1e-3) < 1e-12
    assert abs(rel - math.sqrt((1e-6 + 16e-6) / 3) / math.sqrt((0.25 + 16 + 100) / 3)) < 1e-12


def test_paged_decode_window():
    """Sliding-window decode attends positions [n - window, n): window >= n is
    the full decode; window 1 returns the last token's V for every q head
    (a softmax over one key); tokens outside the window do not matter."""
    rng = np.random.default_rng(12)
    hq, hkv, d, bs, n = 8, 2, 64, 16, 70
    k = rng.standard_normal((n, hkv, d)).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    nb = (n + bs - 1) // bs + 1
    kc, ks = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    vc, vs = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    bt = np.array([[3, 0, 4, 1, 2]], np.int32)
    slots = (bt[0, np.arange(n) // bs] * bs + np.arange(n) % bs).astype(np.int32)
    O.quantize_kv_write_paged(k, v, kc, ks, vc, vs, slots)
    layer = O.LayerCache(kc, ks, vc, vs)
    q = rng.standard_normal((1, hq, d))
    lens = np.array([n])
    full = O.paged_decode(q, layer, bt, lens, 0.125)
    assert np.array_equal(O.paged_decode(q, layer, bt, lens, 0.125, window=n), full)
    assert np.array_equal(O.paged_decode(q, layer, bt, lens, 0.125, window=10 * n), full)
    assert not np.allclose(O.paged_decode(q, layer, bt, lens, 0.125, window=n - 1), full)
    last_v = O.exact_kv(layer, bt[0], n)[1][:, -1]  # [Hkv, D]
    w1 = O.paged_decode(q, layer, bt, lens, 0.125, window=1)[0]
    assert np.allclose(w1, np.repeat(last_v, hq // hkv, axis=0), rtol=1e-12, atol=1e-12)
    # garbage before the window leaves the windowed output unchanged
    w = 23
    before = O.paged_decode(q, layer, bt, lens, 0.125, window=w)
    for p in range(n - w):
        blk, off = bt[0, p // bs], p % bs
        kc[blk, :, off] = 127
        ks[blk, :, off] = 1e3
    assert np.array_equal(O.paged_decode(q, layer, bt, lens, 0.125, window=w), before)
    assert not np.array_equal(O.paged_decode(q, layer, bt, lens, 0.125), full)


def test_paged_verify_window():
    """Verify of a sliding-window layer sees only the last `window` prefix keys:
    window >= prefix is the plain verify, keys before the window do not matter."""
    rng = np.random.default_rng(13)
    hq, hkv, d, bs, p, s = 4, 2, 64, 16, 50, 4
    n = p + s
    k = rng.standard_normal((n, hkv, d)).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    nb = (n + bs - 1) // bs
    kc, ks = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    vc, vs = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    bt = np.arange(nb, dtype=np.int32)[None][:, ::-1].copy()
    slots = (bt[0, np.arange(n) // bs] * bs + np.arange(n) % bs).astype(np.int32)
    O.quantize_kv_write_paged(k, v, kc, ks, vc, vs, slots)
    layer = O.LayerCache(kc, ks, vc, vs)
    q = rng.standard_normal((1, hq, s, d))
    pl = np.array([p])
    full = O.paged_verify(q, layer, bt, pl, 0.125)
    assert np.array_equal(O.paged_verify(q, layer, bt, pl, 0.125, window=p), full)
    w = 20
    before = O.paged_verify(q, layer, bt, pl, 0.125, window=w)
    assert not np.allclose(before, full)
    for pos in range(p - w):
        kc[bt[0, pos // bs], :, pos % bs] = 127
    assert np.array_equal(O.paged_verify(q, layer, bt, pl, 0.125, window=w), before)


def test_paged_verify_window_fresh_drafts_is_the_references_dense_formulation():
    """The reference's window verify (gqa_attention.py:298-313): read the
    prefix window back dense, concatenate the fresh fp16 drafts, run causal
    attention with the S queries at the end.  The oracle's fresh-draft mode
    equals that formulation restated with read_dense and the dense oracle (an
    independent path: keys in fp16 as the reference's reader returns them, so
    the match is to fp16 rounding of the prefix keys), and differs from
    attending the cache-roundtripped drafts."""
    rng = np.random.default_rng(14)
    hq, hkv, d, bs, p, s, w = 4, 2, 64, 16, 70, 5, 24
    n = p + s
    k = (rng.standard_normal((n, hkv, d)) * 2).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    nb = (n + bs - 1) // bs
    kc, ks = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    vc, vs = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    bt = np.arange(nb, dtype=np.int32)[None][:, ::-1].copy()
    slots = (bt[0, np.arange(n) // bs] * bs + np.arange(n) % bs).astype(np.int32)
    O.quantize_kv_write_paged(k, v, kc, ks, vc, vs, slots)
    layer = O.LayerCache(kc, ks, vc, vs)
    q = rng.standard_normal((1, hq, s, d)).astype(np.float16)
    kd, vd = k[None, p:], v[None, p:]  # [1, S, Hkv, D]
    got = O.paged_verify(q, layer, bt, np.array([p]), 0.125, window=w, fresh_drafts=(kd, vd))
    kb, vb = O.read_dense(layer, bt[0], p, window=w)  # [1, Hkv, w, D] fp16
    k_all = np.concatenate([kb[0].transpose(1, 0, 2), k[p:]], axis=0)  # [w + S, Hkv, D]
    v_all = np.concatenate([vb[0].transpose(1, 0, 2), v[p:]], axis=0)
    ref = O.dense_varlen_attention(q[0].transpose(1, 0, 2), k_all, v_all, np.array([0, s]), np.array([0, w + s]),
                                   0.125, causal=True)
    assert np.abs(got[0].transpose(1, 0, 2) - ref).max() < 5e-3
    roundtrip = O.paged_verify(q, layer, bt, np.array([p]), 0.125, window=w)
    assert np.abs(roundtrip - got).max() > 1e-4


@pytest.mark.parametrize("causal", [True, False])
def test_dense_varlen_attention_matches_torch_sdpa(causal):
    """The dense prefill oracle against torch's float64 scaled_dot_product_attention
    with an explicitly built bottom-right causal mask, GQA by repeated KV heads."""
    rng = np.random.default_rng(21)
    hq, hkv, d = 8, 2, 32
    qlens, klens = [5, 1, 9, 7], [5, 4, 20, 7]  # equal, chunked (nq < nk), and a one-token query
    cu_q, cu_k = np.cumsum([0] + qlens), np.cumsum([0] + klens)
    q = rng.standard_normal((cu_q[-1], hq, d))
    k = rng.standard_normal((cu_k[-1], hkv, d))
    v = rng.standard_normal((cu_k[-1], hkv, d))
    got = O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.3, causal)
    for b in range(len(qlens)):
        nq, nk = qlens[b], klens[b]
        qb = torch.from_numpy(q[cu_q[b]:cu_q[b + 1]]).permute(1, 0, 2)
        kb = torch.from_numpy(k[cu_k[b]:cu_k[b + 1]]).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
        vb = torch.from_numpy(v[cu_k[b]:cu_k[b + 1]]).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
        mask = torch.ones(nq, nk, dtype=torch.bool).tril(diagonal=nk - nq) if causal else None
        ref = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask, scale=0.3)
        assert np.allclose(got[cu_q[b]:cu_q[b + 1]], ref.permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)


def test_dense_varlen_attention_window_left_matches_torch_sdpa():
    """window_left: query i (bottom-right aligned) sees its last W keys,
    i - W + 1 .. i, as a torch band mask built with tril / triu; W = 1 is the
    diagonal alone, and the decode-side window of the same layer (the last
    W keys of the row, paged_decode(window=W)) sees the same keys."""
    rng = np.random.default_rng(22)
    hq, hkv, d, w = 4, 2, 16, 5
    qlens, klens = [12, 3], [12, 20]
    cu_q, cu_k = np.cumsum([0] + qlens), np.cumsum([0] + klens)
    q = rng.standard_normal((cu_q[-1], hq, d))
    k = rng.standard_normal((cu_k[-1], hkv, d))
    v = rng.standard_normal((cu_k[-1], hkv, d))
    got = O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.25, True, window_left=w)
    for b in range(2):
        nq, nk = qlens[b], klens[b]
        qb = torch.from_numpy(q[cu_q[b]:cu_q[b + 1]]).permute(1, 0, 2)
        kb = torch.from_numpy(k[cu_k[b]:cu_k[b + 1]]).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
        vb = torch.from_numpy(v[cu_k[b]:cu_k[b + 1]]).permute(1, 0, 2).repeat_interleave(hq // hkv, 0)
        ones = torch.ones(nq, nk, dtype=torch.bool)
        mask = ones.tril(diagonal=nk - nq) & ones.triu(diagonal=nk - nq - w + 1)
        ref = torch.nn.functional.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask, scale=0.25)
        assert np.allclose(got[cu_q[b]:cu_q[b + 1]], ref.permute(1, 0, 2).numpy(), rtol=1e-10, atol=1e-12)
    full = O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.25, True)
    assert np.array_equal(O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.25, True, window_left=100), full)
    one = O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.25, True, window_left=1)
    diag = np.repeat(v[cu_k[1] - qlens[0]:cu_k[1]], hq // hkv, axis=1)  # sequence 0: nk == nq, each its own V
    assert np.allclose(one[:qlens[0]], diag, rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError):
        O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.25, True, window_left=0)


def test_prefill_band_and_decode_window_see_the_same_keys():
    """The last query of a prefill with window_left W attends exactly what the
    decode-side window of W keys attends at that position."""
    rng = np.random.default_rng(23)
    hq, hkv, d, bs, n, w = 4, 2, 32, 8, 40, 9
    k = rng.standard_normal((n, hkv, d)).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    q = rng.standard_normal((n, hq, d)).astype(np.float16)
    nb = n // bs
    kc, ks = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    vc, vs = np.zeros((nb, hkv, bs, d), np.int8), np.ones((nb, hkv, bs), np.float32)
    bt = np.arange(nb, dtype=np.int32)[None]
    O.quantize_kv_write_paged(k, v, kc, ks, vc, vs, np.arange(n, dtype=np.int32))
    layer = O.LayerCache(kc, ks, vc, vs)
    kx, vx = O.exact_kv(layer, bt[0], n)  # the cache's exact values, [Hkv, n, D]
    band = O.dense_varlen_attention(q, kx.transpose(1, 0, 2), vx.transpose(1, 0, 2), np.array([0, n]),
                                    np.array([0, n]), 0.2, True, window_left=w)
    dec = O.paged_decode(q[None, -1], layer, bt, np.array([n]), 0.2, window=w)
    assert np.allclose(band[-1], dec[0], rtol=1e-12, atol=1e-12)
