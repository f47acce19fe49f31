"""GPU parity of the ``superl8`` interface's helpers, through the C ABI:

* ``quantize_i8_rowwise(rotate_last(k))`` holds the K bytes the append kernel
  writes, and the oracle's;
* ``quantize_lloydmax`` + ``pack_indices_lowbit`` hold the K8V3 append's V
  words and norms, and the oracle's; ``unpack`` inverts ``pack``;
* the reference's own two-step K8V3 write recipe (kv_cache.py:587-626),
  replayed with these helpers, leaves the cache byte-identical to the fused
  K8V3 append;
* ``rotate_last`` in fp16 / bf16 / fp32 equals the oracle's rotation rounded
  once; the dequantizers equal the oracle's;
* the dense attention entry points (``attn_int8_decode`` / ``_fwd`` /
  ``_varlen``) are within tolerance of float64 attention."""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops, shim

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _installed():
    saved = {k: sys.modules.get(k) for k in shim._NAMES}
    shim.install()
    yield
    for k, v in saved.items():
        if v is None:
            sys.modules.pop(k, None)
        else:
            sys.modules[k] = v


def _same(a, b):
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint8), b.view(np.uint8))


def _rows(t, hkv, d, seed, outliers=True):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((t, hkv, d)).astype(np.float32)
    if outliers:
        x[..., rng.choice(d, 2, replace=False)] *= 20.0
    x[0, 0] = 0.0                 # an all-zero row
    x[1, 0, :] = 0.0
    x[1, 0, 3] = 65504.0          # the fp16 extremes
    x[1, 0, 5] = -65504.0
    return x.astype(np.float16)


def _np(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rotate_then_rowwise_int8_is_the_append_k_bytes(d):
    import superl8
    from superl8.quant.rotation import rotate_last

    t, hkv, bs = 40, 4, 16
    k = _rows(t, hkv, d, 1)
    v = _rows(t, hkv, d, 2)
    nblk = (t + bs - 1) // bs
    kc = torch.zeros((nblk, hkv, bs, d), dtype=torch.int8, device=DEV)
    ks = torch.ones((nblk, hkv, bs), device=DEV)
    vc, vs = torch.zeros_like(kc), torch.ones_like(ks)
    slots = torch.arange(t, dtype=torch.int32, device=DEV)
    kt, vt = torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV)
    ops.quantize_kv_write_paged(kt, vt, kc, ks, vc, vs, slots)
    k_rot = rotate_last(kt)
    q, s = superl8.quantize_i8_rowwise(k_rot.reshape(-1, d))
    rows = O.flat_rows(np.arange(t), hkv, bs).reshape(-1)
    assert _same(_np(q), _np(kc).reshape(-1, d)[rows]) and _same(_np(s), _np(ks).reshape(-1)[rows])
    oq, os_ = O.quantize_i8_rowwise(O.rotate_last(k))
    assert _same(_np(q), oq.reshape(-1, d)) and _same(_np(s), os_.reshape(-1))
    # V: RTN without rotation; and quantize_kv_cache of [B, Hkv, N, D] views
    qv, sv = superl8.quantize_i8_rowwise(vt)
    assert _same(_np(qv).reshape(-1, d), _np(vc).reshape(-1, d)[rows])
    kb, vb = kt.transpose(0, 1)[None], vt.transpose(0, 1)[None]  # [1, Hkv, T, D] strided views
    k8, k_sc, v8, v_sc = superl8.quantize_kv_cache(kb, vb)
    assert _same(_np(k8)[0].transpose(1, 0, 2), oq) and _same(_np(k_sc)[0].T, os_)
    assert _same(_np(v8)[0].transpose(1, 0, 2), _np(qv)) and _same(_np(v_sc)[0].T, _np(sv))


@pytest.mark.parametrize("d", [128, 256])
def test_lloydmax_and_bitplane_pack_are_the_k8v3_append_bytes(d):
    from superl8.quant.lloydmax import gaussian_codebook, pack_indices_lowbit, quantize_lloydmax, \
        unpack_indices_lowbit

    t, hkv, bs = 40, 4, 16
    k = _rows(t, hkv, d, 3)
    v = _rows(t, hkv, d, 4)
    cb = gaussian_codebook(3, 128, DEV)
    nblk = (t + bs - 1) // bs
    kc = torch.zeros((nblk, hkv, bs, d), dtype=torch.int8, device=DEV)
    ks = torch.ones((nblk, hkv, bs), device=DEV)
    vp = torch.zeros((nblk, hkv, bs, d * 3 // 32), dtype=torch.int32, device=DEV)
    vn = torch.zeros((nblk, hkv, bs, d // 128), device=DEV)
    vt = torch.from_numpy(v).to(DEV)
    ops.quantize_kv_write_paged_k8v3(torch.from_numpy(k).to(DEV), vt, kc, ks, vp, vn, cb,
                                     torch.arange(t, dtype=torch.int32, device=DEV))
    codes, norms, cb2 = quantize_lloydmax(vt, bits=3, block_size=128, dim=-1, codebook=cb)
    assert codes.dtype == torch.uint8 and codes.shape == vt.shape and norms.shape == (t, hkv, d // 128)
    words = pack_indices_lowbit(codes, 3)
    rows = O.flat_rows(np.arange(t), hkv, bs).reshape(-1)
    assert _same(_np(words).reshape(-1, d * 3 // 32), _np(vp).reshape(-1, d * 3 // 32)[rows])
    assert _same(_np(norms).reshape(-1, d // 128), _np(vn).reshape(-1, d // 128)[rows])
    oc, on = O.quantize_lloydmax(v, O.gaussian_codebook(), 128)
    assert _same(_np(codes), oc) and _same(_np(norms), on)
    assert _same(_np(words), O.pack_indices_lowbit(oc, 3))
    assert torch.equal(unpack_indices_lowbit(words, 3, d), codes)


def test_pack_unpack_round_trip_on_every_code():
    from superl8.quant.lloydmax import pack_indices_lowbit, unpack_indices_lowbit

    rng = np.random.default_rng(5)
    codes = rng.integers(0, 8, size=(7, 3, 256)).astype(np.uint8)
    w = pack_indices_lowbit(torch.from_numpy(codes).to(DEV), 3)
    assert _same(_np(w), O.pack_indices_lowbit(codes, 3))
    assert _same(_np(unpack_indices_lowbit(w, 3, 256)), codes)


def test_reference_k8v3_write_recipe_equals_the_fused_append():
    """The reference's K8V3 write, step by step as kv_cache.py:587-626 does
    it (rotate_last -> quantize_i8_rowwise -> scatter at the flat rows;
    quantize_lloydmax -> pack_indices_lowbit -> scatter), through this
    interface, stores exactly what the fused K8V3 append stores."""
    import superl8
    from superl8.quant.lloydmax import gaussian_codebook, pack_indices_lowbit, quantize_lloydmax
    from superl8.quant.rotation import rotate_last

    b, hkv, d, bs, nblk = 24, 8, 128, 16, 12
    rng = np.random.default_rng(6)
    k = torch.from_numpy(_rows(b, hkv, d, 7)).to(DEV)
    v = torch.from_numpy(_rows(b, hkv, d, 8)).to(DEV)
    slots = torch.from_numpy(rng.permutation(nblk * bs)[:b].astype(np.int32)).to(DEV)
    cb = gaussian_codebook(3, 128, DEV)
    shape = (nblk, hkv, bs, d)

    def fresh():
        return (torch.zeros(shape, dtype=torch.int8, device=DEV), torch.ones(shape[:3], device=DEV),
                torch.zeros(shape[:3] + (d * 3 // 32,), dtype=torch.int32, device=DEV),
                torch.zeros(shape[:3] + (1,), device=DEV))

    fused = fresh()
    ops.quantize_kv_write_paged_k8v3(k, v, *fused, cb, slots)
    kc, ks, vp, vn = fresh()
    sm = slots.long()
    blk, off = sm // bs, sm % bs
    rows = ((blk[:, None] * hkv + torch.arange(hkv, device=DEV)[None, :]) * bs + off[:, None]).reshape(-1)
    k_i8, k_sc = superl8.quantize_i8_rowwise(rotate_last(k).reshape(-1, d))
    kc.reshape(-1, d)[rows] = k_i8
    ks.reshape(-1)[rows] = k_sc
    codes, norms, _ = quantize_lloydmax(v, bits=3, block_size=128, dim=-1, codebook=cb)
    packed = pack_indices_lowbit(codes, 3)
    vp.reshape(-1, packed.shape[-1])[rows] = packed.reshape(-1, packed.shape[-1])
    vn.reshape(-1, vn.shape[-1])[rows] = norms.reshape(-1, vn.shape[-1])
    for a, f, name in zip((kc, ks, vp, vn), fused, ("k_cache", "k_scale", "v_packed", "v_norm")):
        assert _same(_np(a), _np(f)), f"{name}: the two-step write differs from the fused append"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_rotate_last_is_the_oracle_rotation_rounded_once(dtype, d):
    from superl8.quant.rotation import hadamard_matrix, rotate_last

    rng = np.random.default_rng(d)
    x32 = (rng.standard_normal((5, 3, d)) * 4).astype(np.float32)
    x = torch.from_numpy(x32).to(dtype)
    exact = O.fwht_f32(x.float().numpy()) * O.rotate_norm_const(d)  # fp32, the oracle's op order
    got = rotate_last(x.to(DEV)).cpu()
    assert got.dtype == dtype and got.shape == x.shape
    want = torch.from_numpy(np.ascontiguousarray(exact)).to(dtype)  # one round-to-nearest-even
    assert torch.equal(got.contiguous().view(torch.uint8), want.contiguous().view(torch.uint8))
    # a rotation by the orthogonal, symmetric matrix the name says
    ref = x.double() @ hadamard_matrix(d, device="cpu", dtype=torch.float64)
    tol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}[dtype]
    assert torch.allclose(got.double(), ref, rtol=tol, atol=tol * ref.abs().max().item())


def test_dequantizers_equal_the_oracle():
    import superl8
    from superl8.quant.lloydmax import dequantize_lloydmax, fake_quant_lloydmax, gaussian_codebook, \
        quantize_lloydmax

    v = torch.from_numpy(_rows(16, 4, 256, 9)).to(DEV)
    cb = gaussian_codebook(3, 128, DEV)
    codes, norms, _ = quantize_lloydmax(v, codebook=cb)
    deq = dequantize_lloydmax(codes, norms, cb, block_size=128, dim=-1)
    assert deq.dtype == torch.float32
    want = O.dequantize_lloydmax(_np(codes), _np(norms), O.gaussian_codebook(), 128)
    assert _same(_np(deq), want)
    fq = fake_quant_lloydmax(v, bits=3, block_size=128)
    assert fq.dtype == torch.float16 and torch.equal(fq, deq.half())
    q, s = superl8.quantize_i8_rowwise(v)
    dq = superl8.quant.dequantize_int8_rowwise(q, s.unsqueeze(-1))
    assert _same(_np(dq), O.dequantize_int8_rowwise(_np(q), _np(s)))


def test_dense_attention_entry_points():
    import superl8

    rng = np.random.default_rng(10)
    b, hq, hkv, n, d = 3, 16, 4, 300, 128
    scale = 1.0 / math.sqrt(d)
    k = rng.standard_normal((b, hkv, n, d)).astype(np.float16)
    v = rng.standard_normal((b, hkv, n, d)).astype(np.float16)
    q1 = rng.standard_normal((b, hq, 1, d)).astype(np.float16)
    kt, vt = torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV)
    out = superl8.attn_int8_decode(torch.from_numpy(q1).to(DEV), kt, vt, scale=scale)
    g = hq // hkv
    for bi in range(b):
        for h in range(hq):
            ref = O._softmax_attend(q1[bi, h].astype(np.float64), k[bi, h // g].astype(np.float64),
                                    v[bi, h // g].astype(np.float64), scale)
            mx, rel = O.attention_errors(_np(out.float())[bi, h], ref)
            assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL
    # causal chunk of 40 queries at the end of 300 keys, as [B, H, S, D] and as varlen
    s = 40
    qs = rng.standard_normal((b, hq, s, d)).astype(np.float16)
    out = _np(superl8.attn_int8_fwd(torch.from_numpy(qs).to(DEV), kt, vt, causal=True, scale=scale,
                                    window_left=-1).float())
    tq = qs.transpose(0, 2, 1, 3).reshape(b * s, hq, d)
    tk, tv = k.transpose(0, 2, 1, 3).reshape(b * n, hkv, d), v.transpose(0, 2, 1, 3).reshape(b * n, hkv, d)
    cu_q, cu_k = np.arange(0, (b + 1) * s, s), np.arange(0, (b + 1) * n, n)
    ref = O.dense_varlen_attention(tq, tk, tv, cu_q, cu_k, scale, causal=True)
    mx, rel = O.attention_errors(out.transpose(0, 2, 1, 3).reshape(b * s, hq, d), ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL
    to = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV)  # noqa: E731
    outv = superl8.attn_int8_varlen(to(tq), to(tk), to(tv), to(cu_q.astype(np.int32)), to(cu_k.astype(np.int32)),
                                    s, n, causal=True, scale=scale)
    mx, rel = O.attention_errors(_np(outv.float()), ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL
