"""GPU parity of the dense prefill attention over fresh fp16 K / V (varlen
batched, the role of superl8.attn_int8_varlen / attn_int8_fwd at
gqa_attention.py:81-128) against the float64 oracle, through the C ABI.
Tolerance as for decode: max(|out-ref| / max(1,|ref|)) <= 2e-3 and relative
RMS <= 1e-3."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from superl8_serve_amd import ops

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _t(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def _close(out, ref, what):
    mx, rel = O.attention_errors(out, ref)
    assert mx <= O.MAX_ABS_TOL and rel <= O.REL_RMS_TOL, f"{what}: max err {mx:.3e}, rel rms {rel:.3e}"


def _case(seed, hq, hkv, d, qlens, klens, outliers=2):
    rng = np.random.default_rng(seed)
    cu_q, cu_k = np.cumsum([0] + list(qlens)).astype(np.int32), np.cumsum([0] + list(klens)).astype(np.int32)
    q = rng.standard_normal((cu_q[-1], hq, d)).astype(np.float32)
    k = rng.standard_normal((cu_k[-1], hkv, d)).astype(np.float32)
    v = rng.standard_normal((cu_k[-1], hkv, d)).astype(np.float32)
    if outliers:
        ch = rng.choice(d, outliers, replace=False)
        q[..., ch] *= 20.0
        k[..., ch] *= 20.0
        v[..., ch] *= 20.0
    return q.astype(np.float16), k.astype(np.float16), v.astype(np.float16), cu_q, cu_k


@pytest.mark.parametrize("hq,hkv,d,qlens,klens,causal", [
    (8, 2, 128, [1, 33, 500, 130], [1, 33, 500, 130], True),     # self-attention prefill, ragged
    (8, 2, 128, [40, 1, 200], [300, 77, 200], True),             # chunks after cached prefixes (nq < nk)
    (16, 16, 64, [65, 3], [65, 3], True),                        # G = 1
    (32, 2, 128, [90, 17], [90, 17], True),                      # G = 16
    (4, 2, 256, [70, 129], [70, 200], True),                     # head_dim 256
    (8, 2, 128, [50, 7], [80, 7], False),                        # not causal
    (8, 2, 128, [2048], [2048], True),                           # one long sequence
])
def test_attn_varlen(hq, hkv, d, qlens, klens, causal):
    q, k, v, cu_q, cu_k = _case(700 + d + len(qlens), hq, hkv, d, qlens, klens)
    scale = 1.0 / np.sqrt(d)
    out = ops.attn_varlen(_t(q), _t(k), _t(v), _t(cu_q), _t(cu_k), max(qlens), max(klens), causal=causal, scale=scale)
    torch.cuda.synchronize()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, scale, causal)
    _close(out.float().cpu().numpy(), ref, "attn_varlen")


def test_attn_fwd_equals_varlen_and_oracle():
    """The [B, H, S, D] wrapper (attn_int8_fwd's layout) on strided views."""
    rng = np.random.default_rng(731)
    b, hq, hkv, sq, sk, d = 3, 8, 2, 40, 100, 128
    q = rng.standard_normal((b, sq, hq, d)).astype(np.float16)
    k = rng.standard_normal((b, sk, hkv, d)).astype(np.float16)
    v = rng.standard_normal((b, sk, hkv, d)).astype(np.float16)
    out = ops.attn_fwd(_t(q).transpose(1, 2), _t(k).transpose(1, 2), _t(v).transpose(1, 2), causal=True, scale=0.1)
    torch.cuda.synchronize()
    cu_q = np.arange(0, (b + 1) * sq, sq, dtype=np.int32)
    cu_k = np.arange(0, (b + 1) * sk, sk, dtype=np.int32)
    ref = O.dense_varlen_attention(q.reshape(b * sq, hq, d), k.reshape(b * sk, hkv, d), v.reshape(b * sk, hkv, d),
                                   cu_q, cu_k, 0.1, True).reshape(b, sq, hq, d).transpose(0, 2, 1, 3)
    _close(out.float().cpu().numpy(), ref, "attn_fwd")


def test_attn_varlen_writes_only_own_tokens():
    """A query that sees no key (nq > nk, causal) is zero, and tokens of other
    sequences are left as they are in a preallocated layout."""
    q, k, v, cu_q, cu_k = _case(741, 8, 2, 128, [6, 10], [3, 10], outliers=0)
    out = ops.attn_varlen(_t(q), _t(k), _t(v), _t(cu_q), _t(cu_k), 10, 10, causal=True, scale=0.1)
    torch.cuda.synchronize()
    o = out.float().cpu().numpy()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.1, True)
    assert np.all(o[:3] == 0) and np.all(ref[:3] == 0)  # queries 0..2 of sequence 0 see no key
    _close(o, ref, "nq > nk")


@pytest.mark.parametrize("d,qlens,klens,w", [
    (128, [300, 33, 7], [300, 33, 7], 64),      # band inside long sequences, shorter ones
    (128, [100, 40], [400, 40], 1),             # only the diagonal key; a chunk after a prefix
    (64, [257], [257], 32),                     # band edge off a 32-key tile
    (256, [90, 130], [200, 130], 100),          # head_dim 256
])
def test_attn_varlen_window_left(d, qlens, klens, w):
    q, k, v, cu_q, cu_k = _case(750 + d + w, 8, 2, d, qlens, klens)
    scale = 1.0 / np.sqrt(d)
    out = ops.attn_varlen(_t(q), _t(k), _t(v), _t(cu_q), _t(cu_k), max(qlens), max(klens), causal=True, scale=scale,
                          window_left=w)
    torch.cuda.synchronize()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, scale, True, window_left=w)
    _close(out.float().cpu().numpy(), ref, f"window_left {w}")


def test_attn_varlen_band_long_sequence_g16():
    """head_dim 128 with a band inside a long sequence and 16 q heads per KV
    head (128-row workgroups of 8 positions): the band's lower edge moves
    across the tiles of every block."""
    q, k, v, cu_q, cu_k = _case(771, 32, 2, 128, [1000, 70], [1000, 300])
    scale = 1.0 / np.sqrt(128)
    out = ops.attn_varlen(_t(q), _t(k), _t(v), _t(cu_q), _t(cu_k), 1000, 1000, causal=True, scale=scale,
                          window_left=100)
    torch.cuda.synchronize()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, scale, True, window_left=100)
    _close(out.float().cpu().numpy(), ref, "band, G = 16")


@pytest.mark.parametrize("window_left", [None, 50])
def test_attn_varlen_unaligned_q(window_left):
    """q rows that are not 16-byte aligned (a view 4 elements into each row)
    take the 16-row kernel; the result is the same attention."""
    q, k, v, cu_q, cu_k = _case(781, 8, 2, 128, [120, 9], [200, 9])
    qbig = np.zeros((q.shape[0], q.shape[1], 136), np.float16)
    qbig[:, :, 4:132] = q
    qv = _t(qbig)[:, :, 4:132]
    assert qv.data_ptr() % 16 != 0
    out = ops.attn_varlen(qv, _t(k), _t(v), _t(cu_q), _t(cu_k), 120, 200, causal=True, scale=0.1,
                          window_left=window_left)
    torch.cuda.synchronize()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.1, True, window_left=window_left)
    _close(out.float().cpu().numpy(), ref, f"unaligned q, window {window_left}")


def test_attn_varlen_wide_window_equals_plain_causal():
    q, k, v, cu_q, cu_k = _case(761, 8, 2, 128, [200, 50], [200, 90])
    args = (_t(q), _t(k), _t(v), _t(cu_q), _t(cu_k), 200, 200)
    a = ops.attn_varlen(*args, causal=True, scale=0.1, window_left=1000)
    b = ops.attn_varlen(*args, causal=True, scale=0.1)
    torch.cuda.synchronize()
    ref = O.dense_varlen_attention(q, k, v, cu_q, cu_k, 0.1, True)
    _close(a.float().cpu().numpy(), ref, "wide window")
    _close(b.float().cpu().numpy(), ref, "plain")
